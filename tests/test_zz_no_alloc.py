"""The allocation-free forward (pf_gdn_exec_static) against the workspace forward (pf_gdn_exec),
through the C ABI on the GPU.

Both run the same kernels on the same inputs, so their outputs must be bit-identical.  Two calls
in a row, the second on a smaller input (the static scratch keeps the first call's contents, and
nothing of them may leak into the second), then an input larger than the scratch, which must be
refused with PF_ERR_SCRATCH before anything is launched (the outputs keep their sentinel).
"""
import numpy as np
import pytest
import torch

from conftest import announce
from pto_fuser_amd import _hip
from pto_fuser_amd.forwards import make_delta_inputs
from pto_fuser_amd.ops import gdn_workspace

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
C, DK, DV = 64, 128, 128


def _static(d, o, hf, B, H, T, code):
    lib = _hip.load()
    return lib.pf_gdn_exec_static(
        _hip.ptr(d["q"]), _hip.ptr(d["k"]), _hip.ptr(d["v"]), _hip.ptr(d["beta"]),
        _hip.ptr(d["g"]), _hip.ptr(d["h0"]), _hip.ptr(o), _hip.ptr(hf), B, H, T, C, DK, DV, code,
        DK ** -0.5, _hip.current_stream_handle(DEV))


def _with_workspace(d, o, hf, B, H, T, dtype, code):
    lib = _hip.load()
    ws = gdn_workspace(B, H, T, C, DK, DV, dtype, DEV)
    return lib.pf_gdn_exec(
        _hip.ptr(d["q"]), _hip.ptr(d["k"]), _hip.ptr(d["v"]), _hip.ptr(d["beta"]),
        _hip.ptr(d["g"]), _hip.ptr(d["h0"]), _hip.ptr(o), _hip.ptr(hf), B, H, T, C, DK, DV, code,
        DK ** -0.5, ws.handle, _hip.current_stream_handle(DEV))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_static_forward_matches_workspace_forward(dtype):
    code = _hip.PF_DTYPE_BF16 if dtype == torch.bfloat16 else _hip.PF_DTYPE_F32
    # bf16 starts at the headline shape (4096 chunks: the 32-column scan, most of the scratch);
    # each later call is smaller
    calls = ((4, 16, 4096, 20),) if dtype == torch.bfloat16 else ()
    for B, H, T, seed in calls + ((2, 8, 1024, 21), (1, 4, 256, 22)):
        announce(f"pf_gdn_exec_static vs pf_gdn_exec {dtype} B{B} H{H} T{T}")
        d = make_delta_inputs(B, H, T, kind="gdn", dtype=dtype, seed=seed, h0_std=0.02, device=DEV)
        outs = {}
        for name in ("static", "workspace"):
            o = torch.full((B, H, T, DV), float("nan"), device=DEV)
            hf = torch.full((B, H, DK, DV), float("nan"), device=DEV)
            st = (_static(d, o, hf, B, H, T, code) if name == "static"
                  else _with_workspace(d, o, hf, B, H, T, dtype, code))
            _hip.check(f"pf_gdn_exec{'_static' if name == 'static' else ''}", st)
            torch.cuda.synchronize()
            outs[name] = (o.cpu().numpy(), hf.cpu().numpy())
        assert np.isfinite(outs["static"][0]).all() and np.isfinite(outs["static"][1]).all()
        assert np.array_equal(outs["static"][0], outs["workspace"][0])
        assert np.array_equal(outs["static"][1], outs["workspace"][1])


def test_static_forward_refuses_inputs_beyond_its_scratch():
    B, H, T = 8, 16, 4096                                 # 8192 chunks: past the 40 MiB scratch
    announce(f"pf_gdn_exec_static oversized B{B} H{H} T{T}")
    d = make_delta_inputs(B, H, T, kind="gdn", dtype=torch.bfloat16, seed=23, device=DEV)
    o = torch.full((B, H, T, DV), -7.0, device=DEV)
    hf = torch.full((B, H, DK, DV), -7.0, device=DEV)
    st = _static(d, o, hf, B, H, T, _hip.PF_DTYPE_BF16)
    torch.cuda.synchronize()
    assert st == _hip.PF_ERR_SCRATCH, st
    assert "static scratch" in _hip.status_text(st)
    assert bool((o == -7.0).all()) and bool((hf == -7.0).all())
