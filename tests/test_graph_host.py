"""Graph-replay and fusion-decision host contracts (no device) — reference tests/test_graph.py
and the FusionDecision part of tests/test_fusion.py."""
import pytest

from pto_fuser_amd import FusionDecision, GraphReplayExecutor, capture_mode, format_fusion_decisions
from pto_fuser_amd import registry as reg


def test_capture_mode_toggles_and_restores():
    assert reg._CAPTURE_MODE is False
    with capture_mode():
        assert reg._CAPTURE_MODE is True and reg.in_capture_mode()
    assert reg._CAPTURE_MODE is False


def test_capture_mode_restores_on_exception():
    with pytest.raises(RuntimeError):
        with capture_mode():
            raise RuntimeError("boom")
    assert reg._CAPTURE_MODE is False


def test_capture_mode_nests():
    with capture_mode():
        with capture_mode():
            assert reg._CAPTURE_MODE is True
        assert reg._CAPTURE_MODE is True
    assert reg._CAPTURE_MODE is False


def test_replay_before_capture_raises():
    with pytest.raises(RuntimeError, match="capture()"):
        GraphReplayExecutor().replay({})


def test_decision_kept_only_if_gated_det_and_faster():
    keep = FusionDecision("s", "k", gated_ok=True, deterministic=True, faster=True, kept=True,
                          t_staged_ms=1.0, t_fused_ms=0.5, frob=0.0, detail="")
    assert keep.kept and abs(keep.speedup - 2.0) < 1e-9 and "FUSE" in str(keep)
    drop = FusionDecision("s", "k", gated_ok=True, deterministic=False, faster=True, kept=False,
                          t_staged_ms=1.0, t_fused_ms=0.5, frob=0.0, detail="")
    assert not drop.kept and "stage" in str(drop)
    assert "1/2 stages fused" in format_fusion_decisions([keep, drop])


def test_opaque_registry_contract():
    r = reg.default_registry()
    assert r.keys() == ["tri_inv_rec_unroll"]
    with pytest.raises(ValueError):
        r.register("tri_inv_rec_unroll", factory=None, lowering=None, contract=None)
    with pytest.raises(KeyError):
        r.run("nope", [], {})
