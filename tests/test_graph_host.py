"""Host-side contracts of graph recording and fusion decisions (no device).

capture_mode counts nesting depth; the recording executor runs every step inside it; replay
refuses to run without a graph; a FusionDecision's verdicts are derived from its measurements
and cannot disagree with them."""
import pytest
import torch

from cpu_kernels import cpu_fused_registry
from pto_fuser_amd import (CaptureExecutor, FusionDecision, GraphReplayExecutor, OpaqueContract,
                           OpaqueNode, OpaqueRegistry, Program, capture_mode,
                           format_fusion_decisions)
from pto_fuser_amd import registry as reg


def test_capture_mode_depth():
    assert not reg.in_capture_mode()
    with capture_mode():
        with capture_mode():
            assert reg.in_capture_mode()
        assert reg.in_capture_mode()          # leaving the inner region keeps the outer one
    assert not reg.in_capture_mode()


def test_capture_mode_unwinds_on_error():
    with pytest.raises(KeyError):
        with capture_mode():
            with capture_mode():
                raise KeyError("x")
    assert not reg.in_capture_mode()


def test_recording_executor_runs_steps_in_capture_mode():
    seen = []
    opaque = OpaqueRegistry()
    opaque.register("probe", factory=lambda: None,
                    lowering=lambda raw, ins, p: seen.append(reg.in_capture_mode()) or ins[0] * 2,
                    contract=OpaqueContract([torch.float32], torch.float32))
    prog = Program([OpaqueNode("probe", ["x"], "y")], ["x"], ["y"])
    out = CaptureExecutor(opaque, fused=cpu_fused_registry()).run(prog, {"x": torch.ones(3)})
    assert seen == [True] and torch.equal(out["y"], torch.full((3,), 2.0))
    assert not reg.in_capture_mode()


def test_replay_needs_a_graph():
    with pytest.raises(RuntimeError, match="capture"):
        GraphReplayExecutor().replay({})


@pytest.mark.parametrize("frob,det,staged,fused,kept,why", [
    (1e-4, True, 1.0, 0.5, True, "kept"),
    (5e-2, True, 1.0, 0.5, False, "frob"),
    (1e-4, False, 1.0, 0.5, False, "runs differ"),
    (1e-4, True, 0.5, 1.0, False, "not faster"),
    (5e-2, False, 0.5, 1.0, False, "frob"),
])
def test_decision_verdict_is_derived(frob, det, staged, fused, kept, why):
    d = FusionDecision("stage", "kernel", frob, det, staged, fused)
    assert d.kept is kept and why in d.detail
    assert d.speedup == pytest.approx(staged / fused)
    assert str(d).startswith("FUSE" if kept else "stage")


def test_decision_summary_counts_kept():
    ds = [FusionDecision("a", "k", 0.0, True, 2.0, 1.0), FusionDecision("b", "k", 0.0, True, 1.0, 2.0),
          FusionDecision("c", "k", 0.0, True, 3.0, 1.0, tol=0.0)]
    text = format_fusion_decisions(ds)
    assert text.splitlines()[-1].startswith("1/3 stages fused")
    assert len(text.splitlines()) == 4


def test_opaque_registry_contract():
    r = reg.default_registry()
    assert r.keys() == ["tri_inv_rec_unroll"]
    assert r.contract("tri_inv_rec_unroll").out_dtype == torch.float32
    with pytest.raises(ValueError, match="already registered"):
        r.register("tri_inv_rec_unroll", factory=None, lowering=None, contract=None)
    with pytest.raises(KeyError, match="tri_inv_rec_unroll"):
        r.run("nope", [], {})
