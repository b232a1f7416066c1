"""The reference-side stub of INTEGRATION.md, executed.

The stub (the ``# file: pto_fuser/fused_hip.py`` block) is loaded as the module
``pto_fuser.fused_hip`` with ``pto_fuser.fused`` resolved to ``pto_fuser_amd.fused``, whose
registry classes have the reference's signatures (src/pto_fuser/fused.py:84-162).  Without a GPU:
those signatures, every symbol the stub binds exported with the header's arity, and the stub's
registry opening the prebuilt library and running every recipe's setup and teardown.  On the GPU:
each recipe's launch against the package's own entry points, and a lowered GDN program run
through the stub's registry."""
import ctypes
import dataclasses
import inspect
import os
import re
import sys
import types

import pytest
import torch

from pto_fuser_amd import _build, _hip, fused as amd_fused

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
MARK = "# file: pto_fuser/fused_hip.py"

# src/pto_fuser/fused.py:119-127 (field order) and :102-103 (FusedKernel.__init__)
REF_RECIPE_FIELDS = ["src_dir", "src_file", "defines", "setup_sym", "teardown_sym", "bind",
                     "launch", "contract"]
REF_KERNEL_PARAMS = ["lib", "launch", "setup_sym", "teardown_sym"]
REF_CONTRACT_FIELDS = ["in_slots", "in_dtypes", "out_names", "out_dtype", "notes"]


def _stub_source() -> str:
    text = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    blocks = [b for b in re.findall(r"```python\n(.*?)```", text, flags=re.S) if MARK in b]
    assert len(blocks) == 1, "INTEGRATION.md must hold exactly one stub block"
    return blocks[0]


@pytest.fixture(scope="module")
def stub():
    _build.ensure_built()
    pkg = types.ModuleType("pto_fuser")
    pkg.__path__ = []
    saved = {n: sys.modules.get(n) for n in ("pto_fuser", "pto_fuser.fused", "pto_fuser.fused_hip")}
    sys.modules["pto_fuser"], sys.modules["pto_fuser.fused"] = pkg, amd_fused
    mod = types.ModuleType("pto_fuser.fused_hip")
    sys.modules["pto_fuser.fused_hip"] = mod
    try:
        exec(compile(_stub_source(), "INTEGRATION.md:fused_hip.py", "exec"), mod.__dict__)
        yield mod
    finally:
        for n, m in saved.items():
            if m is None:
                sys.modules.pop(n, None)
            else:
                sys.modules[n] = m


def _header_arity():
    from test_abi import _header_functions
    return _header_functions()


def test_in_repo_registry_has_the_reference_signatures():
    assert [f.name for f in dataclasses.fields(amd_fused._Recipe)] == REF_RECIPE_FIELDS
    assert [f.name for f in dataclasses.fields(amd_fused.FusedContract)] == REF_CONTRACT_FIELDS
    params = list(inspect.signature(amd_fused.FusedKernel.__init__).parameters)[1:]
    assert params == REF_KERNEL_PARAMS
    reg = amd_fused.FusedKernelRegistry()
    assert hasattr(reg, "_recipes") and hasattr(reg, "_cache")
    for m in ("register", "contract", "kernel", "run", "close"):
        assert callable(getattr(reg, m))


def test_stub_binds_only_exported_declared_symbols(stub):
    arity = _header_arity()
    lib = _hip.load()
    for name, (_, argtypes) in stub.SIGNATURES.items():
        assert name in arity, f"{name} is not declared in include/"
        assert len(argtypes) == arity[name], name
        assert hasattr(lib, name), f"{name} is not exported"
    # and the recipes name only bound symbols
    reg = stub.register_hip_recipes(stub.PrebuiltFusedKernelRegistry(), _build.LIB_DIR)
    for key in reg._recipes:
        r = reg._recipes[key]
        assert r.setup_sym in stub.SIGNATURES and r.teardown_sym in stub.SIGNATURES, key


def test_stub_registry_opens_the_library_and_runs_setup_teardown(stub):
    """kernel() on every key: the prebuilt library opened (no compile), bound, setup called;
    close() runs every teardown.  No device work: the fused-forward setups return empty
    handles, the stage setups NULL."""
    reg = stub.register_hip_recipes(stub.PrebuiltFusedKernelRegistry(), _build.LIB_DIR)
    assert {"gdn_forward", "kda_forward", "chunk_h_scan", "kkt_gated_native_v2",
            "gated_qk_native_v2", "qkv_flash_native_v2"} <= set(reg._recipes)
    params = {"B": 1, "H": 2, "T": 128, "C": 64, "nc": 2, "causal": True}
    kernels = {key: reg.kernel(key, params) for key in reg._recipes}
    assert reg.kernel("gdn_forward", params) is kernels["gdn_forward"]     # cached per shape
    assert reg.kernel("gdn_forward", dict(params, T=256)) is not kernels["gdn_forward"]
    assert kernels["gdn_forward"]._ws and kernels["kda_forward"]._ws
    assert not kernels["chunk_h_scan"]._ws
    lib = kernels["gdn_forward"]._lib
    assert os.path.samefile(lib._name, _hip.lib_path())
    # an unsupported shape is refused by reserve before any allocation
    assert lib.pf_gdn_reserve(kernels["gdn_forward"]._ws, 1, 1, 100, 64, 128, 128, 1) == -1
    assert lib.pf_kda_reserve(kernels["kda_forward"]._ws, 1, 1, 96, 64, 128, 128, 1) == -1
    reg.close()
    assert not reg._cache


def test_reserve_rejects_a_null_handle():
    lib = _hip.load()
    assert lib.pf_gdn_reserve(None, 1, 1, 128, 64, 128, 128, 1) == _hip.PF_ERR_ARG
    ws = lib.pf_gdn_create()
    assert ws
    lib.pf_gdn_teardown(ctypes.c_void_p(ws))
    lib.pf_kda_teardown(None)


# ---- on the GPU ---------------------------------------------------------------------------
DEV = "cuda:0"


def _announce(what):
    from conftest import announce
    announce(what)


@pytest.mark.gpu
def test_stub_forward_launches_equal_the_package(stub):
    from pto_fuser_amd import gdn_chunk_forward, kda_chunk_forward
    B, H, T, D = 2, 3, 256, 128
    _announce(f"integration stub forwards B{B} H{H} T{T}")
    gen = torch.Generator(device=DEV).manual_seed(11)
    q, k, v = (torch.randn(B, H, T, D, device=DEV, generator=gen).to(torch.bfloat16)
               for _ in range(3))
    k = torch.nn.functional.normalize(k.float(), dim=-1).to(torch.bfloat16)
    beta = torch.rand(B, H, T, device=DEV, generator=gen)
    g = -torch.rand(B, H, T, device=DEV, generator=gen) * 0.1
    gk = -torch.rand(B, H, T, D, device=DEV, generator=gen) * 0.1
    reg = stub.register_hip_recipes(stub.PrebuiltFusedKernelRegistry(), _build.LIB_DIR)
    p = {"B": B, "H": H, "T": T, "C": 64}
    for key, gate, ref_fn in (("gdn_forward", g, gdn_chunk_forward),
                              ("gdn_forward", None, gdn_chunk_forward),
                              ("kda_forward", gk, kda_chunk_forward)):
        o, h = reg.run(key, [q, k, v, beta, gate], p)
        o_ref, h_ref = ref_fn(q, k, v, beta, gate)
        torch.cuda.synchronize()
        assert torch.equal(o, o_ref) and torch.equal(h, h_ref), key
    reg.close()


@pytest.mark.gpu
def test_stub_stage_launches_equal_the_package(stub):
    from pto_fuser_amd import ops
    _announce("integration stub stage kernels")
    gen = torch.Generator(device=DEV).manual_seed(12)
    bf = torch.bfloat16
    reg = stub.register_hip_recipes(stub.PrebuiltFusedKernelRegistry(), _build.LIB_DIR)
    # scan
    B, nc, C, H, D = 1, 3, 64, 2, 128
    w, u, k = (0.1 * torch.randn(B, nc, C, H, D, device=DEV, generator=gen)).to(bf), \
        (0.1 * torch.randn(B, nc, C, H, D, device=DEV, generator=gen)).to(bf), \
        (0.1 * torch.randn(B, nc, C, H, D, device=DEV, generator=gen)).to(bf)
    decay = torch.rand(B, H, nc, device=DEV, generator=gen)
    h_out, final = reg.run("chunk_h_scan", [w, u, k, decay], {"B": B, "H": H, "nc": nc})
    ref_h, ref_f = ops.chunk_scan(w, u, k, decay, out_dtype=bf)
    # native chunk stages
    M = 6
    a, b, vv = (torch.randn(M, C, D, device=DEV, generator=gen).to(bf) for _ in range(3))
    gn = -torch.rand(M, C, device=DEV, generator=gen).cumsum(-1) * 0.05
    bn = torch.rand(M, C, device=DEV, generator=gen)
    (L,) = reg.run("kkt_gated_native_v2", [a, gn, bn], {"nc": M, "H": 1})
    ref_L = ops.gated_qk(a, a, gn, bn, chunk_size=C, causal=False, out_dtype=bf)
    (o,) = reg.run("qkv_flash_native_v2", [a, b, vv, gn, bn], {"nc": M, "H": 1})
    ref_o = ops.qkv_flash(a, b, vv, gn, bn, chunk_size=C)
    A = torch.randn(M, C, C, device=DEV, generator=gen).tril(-1) * 0.1
    T = stub.tri_inv_lowering(_hip.load())(None, [A], {})
    torch.cuda.synchronize()
    assert torch.equal(h_out, ref_h) and torch.equal(final, ref_f)
    assert torch.equal(L, ref_L) and torch.equal(o, ref_o)
    assert torch.equal(T, ops.tri_inv(A))
    reg.close()


@pytest.mark.gpu
def test_lowered_program_runs_on_the_stub_registry(stub):
    """The compile stack's lowered GDN program (chunk_h_scan, kkt_gated_native_v2,
    qkv_flash_native_v2) executed with the stub's registry in place of the package's."""
    from pto_fuser_amd import Features, StagedExecutor, compile_program, frob_rel
    from pto_fuser_amd.forwards import build_gdn_program, make_gdn_inputs, prepare_gdn_bindings
    B, H, nc, C, D = 1, 4, 2, 64, 128
    _announce("integration stub lowered program")
    inp = make_gdn_inputs(B, H, nc, C, D, device=DEV, seed=13)
    binds = prepare_gdn_bindings(inp["q"], inp["k"], inp["v"], inp["beta"], inp["g_in"])
    prog = compile_program(build_gdn_program(B, H, nc, C, D, D ** -0.5), Features(B, H, nc, C, D),
                           verify=False).program
    reg = stub.register_hip_recipes(stub.PrebuiltFusedKernelRegistry(), _build.LIB_DIR)
    got = StagedExecutor(fused=reg).run(prog, binds)["o"]
    ref = StagedExecutor().run(prog, binds)["o"]
    torch.cuda.synchronize()
    err = frob_rel(got, ref)
    print(f"stub vs package lowered program: frob {err:.2e}")
    assert err < 1e-2
    reg.close()
