"""Cost model, policy and compile driver without verification (no device)
(reference tests/test_compile.py; the lowered-kernel contract of its lines 77-98 is kept)."""
import torch

from pto_fuser_amd import (CostModel, EinsumNode, Features, FusedNode, Policy, canonicalize,
                           compile_program)
from pto_fuser_amd.cost import CU_COUNT, HBM_EFFECTIVE_BPS
from pto_fuser_amd.forwards import build_gdn_program, build_kda_program


def _gdn():
    return build_gdn_program(1, 16, 8, 128, 128, 128 ** -0.5)


def _kda():
    return build_kda_program(1, 16, 8, 128, 128, 128 ** -0.5)


def test_features_derived():
    f = Features(1, 16, 8, 128, 128)
    assert f.T == 8 * 128 and f.M == 16 * 8 and f.N == 16
    assert f.dtype == torch.bfloat16 and f.esize == 2
    assert Features(1, 1, 1, 64, 128, dtype=torch.float32).esize == 4


def test_regime_is_seeded_for_256_cus():
    # fewer chunk workgroups than CUs -> launch-bound
    assert Features(1, 16, 8, 128, 128).regime == "launch-bound"          # M = 128
    # chunk stages fill the chip but the scan (N x D/32 workgroups) does not
    assert Features(1, 16, 64, 64, 128).regime == "crossover"             # M = 1024, N*4 = 64
    # the headline workload: 64 chains x 4 slices = 256 scan workgroups = one per CU
    assert Features(4, 16, 64, 64, 128).regime == "bandwidth-bound"
    assert CU_COUNT == 256 and HBM_EFFECTIVE_BPS < 8e12


def test_cost_predictions_worth_trying():
    cm, f = CostModel(), Features(1, 16, 8, 128, 128)
    for name in ("enable-direct-reads", "enable-fused-store", "lower-resident-scan",
                 "lower-perdim-scan", "fuse-contraction-epilogue", "fuse-chunk-o-flash",
                 "fuse-perdim-chunk-o-flash", "fuse-gdn-forward", "fuse-kda-forward"):
        assert cm.predict(name, f).worth_trying, name
    assert not cm.predict("unknown", f).worth_trying


def test_resident_scan_benefit_grows_with_chunks():
    cm = CostModel()
    short = cm.predict("lower-resident-scan", Features(1, 16, 4, 64, 128)).benefit
    long = cm.predict("lower-resident-scan", Features(1, 16, 64, 64, 128)).benefit
    assert long > 10 * short > 0


def test_cost_v2_shape_gate():
    cm = CostModel()
    assert cm.predict("fuse-contraction-epilogue", Features(1, 4, 8, 128, 128)).v2 is True
    assert cm.predict("fuse-contraction-epilogue", Features(1, 4, 8, 16, 64)).v2 is False


def test_policy_orders_fusions_before_reads():
    names = [p.name for p in Policy().pipeline(canonicalize(_gdn()), Features(1, 16, 8, 128, 128))]
    assert "lower-perdim-scan" not in names
    assert names.index("lower-resident-scan") < names.index("enable-direct-reads")
    assert names.index("fuse-chunk-o-flash") < names.index("fuse-contraction-epilogue")
    assert names.index("fuse-contraction-epilogue") < names.index("enable-direct-reads")


def test_policy_prunes_by_match():
    names = [p.name for p in Policy().pipeline(canonicalize(_kda()), Features(1, 16, 8, 128, 128))]
    assert "lower-perdim-scan" in names and "fuse-contraction-epilogue" in names
    assert "lower-resident-scan" not in names


def test_compile_gdn_unverified():
    res = compile_program(_gdn(), Features(1, 16, 8, 128, 128), verify=False)
    kernels = {n.kernel for n in res.program.nodes if isinstance(n, FusedNode)}
    assert kernels == {"chunk_h_scan", "kkt_gated_native_v2", "qkv_flash_native_v2"}
    assert all(n.read_mode == "auto" for n in res.program.nodes if isinstance(n, EinsumNode))
    assert not res.report.verified
    assert len(res.report.kept) == len(res.report.records) == 5


def test_compile_kda_unverified():
    res = compile_program(_kda(), Features(1, 16, 8, 128, 128), verify=False)
    kernels = {n.kernel for n in res.program.nodes if isinstance(n, FusedNode)}
    assert kernels == {"chunk_h_scan", "qkvp_flash_native_v2"}
    assert len(res.report.kept) == 4


def test_compile_without_bindings_never_verifies():
    res = compile_program(_gdn(), Features(1, 16, 8, 128, 128), verify=True, bindings=None)
    assert not res.report.verified and len(res.report.kept) == 5


def test_report_str_is_readable():
    text = str(compile_program(_gdn(), Features(1, 16, 8, 128, 128), verify=False).report)
    assert "transforms kept" in text and "lower-resident-scan" in text
