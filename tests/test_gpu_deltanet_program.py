"""The DeltaNet multi-output program on the HIP path (the reference's worked example,
src/pto_fuser/forwards/deltanet.py:23-99, and its device test tests/test_forwards_npu.py:22-43).

``build_deltanet_program`` returns all seven intermediates — A, T, W, U, v_new, h_state and o —
and runs here on the device registries: the triangular inverse through ``pf_tri_inv_exec``, the
contractions on the device.  Each output is gated against ``deltanet_reference`` (the fp64
oracle on the same dtype-rounded inputs) at the reference's frob_rel < 2e-2 for bf16 work and
1e-4 for fp32 work, and two runs must be bit-identical (the reference's determinism gate).  The
scan stage is also run on its own kernel (``pf_scan_exec`` with a unit decay) over the program's
W, U and k, and must reproduce the program's h_state and v_new.
"""
import numpy as np
import pytest
import torch

from conftest import announce, record_error
from oracle.gdn_oracle import deltanet_reference
from pto_fuser_amd import StagedExecutor, chunk_scan, gate_determinism
from pto_fuser_amd.forwards import DELTANET_OUTPUTS, build_deltanet_program, make_inputs

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
B, H, nc, C, D = 1, 2, 3, 64, 128        # the reference test's shape


@pytest.mark.parametrize("work,tol", [(torch.bfloat16, 2e-2), (torch.float32, 1e-4)])
def test_deltanet_program_seven_outputs(work, tol):
    name = str(work).replace("torch.", "")
    announce(f"DeltaNet program {name} B{B} H{H} nc{nc} C{C} D{D}")
    inp = make_inputs(B, H, nc, C, D, device=DEV, dtype=work, seed=0)
    prog = build_deltanet_program(B, H, nc, C, D, D ** -0.5, work=work)
    ex = StagedExecutor()
    got = ex.run(prog, inp)
    torch.cuda.synchronize()
    T = nc * C
    x = {n: t.double().cpu().numpy() for n, t in inp.items()}
    ref = deltanet_reference(x["q"].reshape(B, H, T, D), x["k"].reshape(B, H, T, D),
                             x["v"].reshape(B, H, T, D), x["beta"].reshape(B, H, T), C=C,
                             dtype=np.float64)
    for out in DELTANET_OUTPUTS:
        g = got[out].double().cpu().numpy()
        assert g.shape == ref[out].shape, (out, g.shape, ref[out].shape)
        e = record_error(f"DeltaNet program {name}", out, g, ref[out], f"frob <= {tol}")
        assert e["frob"] < tol, (out, e)
    det = gate_determinism(lambda: ex.run(prog, inp))
    assert det.passed, str(det)


def test_deltanet_scan_stage_on_its_kernel():
    """h_state and v_new of the fp32 program, recomputed by the resident-state scan kernel from the
    program's own W, U and k (decay 1: DeltaNet has no gate)."""
    announce(f"DeltaNet scan stage fp32 B{B} H{H} nc{nc} C{C} D{D}")
    work = torch.float32
    inp = make_inputs(B, H, nc, C, D, device=DEV, dtype=work, seed=1)
    got = StagedExecutor().run(build_deltanet_program(B, H, nc, C, D, D ** -0.5, work=work), inp)
    tok = lambda t: t.permute(0, 2, 3, 1, 4).contiguous()      # [B,H,nc,C,D] -> [B,nc,C,H,D]
    decay = torch.ones(B, H, nc, device=DEV)
    h_out, final = chunk_scan(tok(got["W"]), tok(got["U"]), tok(inp["k"]), decay)
    h_state = h_out.permute(0, 2, 1, 3, 4)                      # [B,nc,H,D,D] -> [B,H,nc,D,D]
    v_new = got["U"] - got["W"] @ h_state
    torch.cuda.synchronize()
    for out, val in (("h_state", h_state), ("v_new", v_new)):
        e = record_error("DeltaNet scan stage fp32", out, val.cpu().numpy(),
                         got[out].cpu().numpy(), "max rel <= 1e-4")
        assert e["rel"] <= 1e-4, (out, e)
