"""Test setup: make the package and the oracle importable without an install, register the
``gpu`` marker, and skip GPU tests cleanly when no HIP device is visible."""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "pto-fuser_amd"))
sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP device (MI355X) and the built library")


def pytest_collection_modifyitems(config, items):
    try:
        import torch
        has_gpu = torch.cuda.is_available()
    except Exception:                       # pragma: no cover - torch missing
        has_gpu = False
    if has_gpu:
        return
    skip = pytest.mark.skip(reason="no HIP device visible")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


def announce(msg: str) -> None:
    """Name the case before a GPU step (flushed, so a box that dies still shows it)."""
    print(f"[gpu-case] {msg}", flush=True)


# (case, output, max abs err, max rel err (max|x - r| / max|r|), frob rel err, tolerance text)
_ERRORS = []


def record_error(case: str, output: str, got, ref, tol: str = "") -> dict:
    """Record the error magnitudes of one parity comparison; the session summary prints them
    all (shown by `pytest -q` too), so a run's log shows how close each case came to its bound."""
    import numpy as np
    g = np.asarray(got, np.float64)
    r = np.asarray(ref, np.float64)
    d = np.abs(g - r)
    e = {"abs": float(d.max()) if d.size else 0.0,
         "rel": float(d.max() / max(np.abs(r).max(), 1e-30)) if d.size else 0.0,
         "frob": float(np.linalg.norm(g - r) / max(np.linalg.norm(r), 1e-30))}
    _ERRORS.append((case, output, e["abs"], e["rel"], e["frob"], tol))
    return e


def pytest_terminal_summary(terminalreporter, exitstatus, config):
    if not _ERRORS:
        return
    tr = terminalreporter
    tr.write_sep("-", "parity error magnitudes (max abs | max rel | frob rel)")
    for case, out, a, r, f, tol in _ERRORS:
        tr.write_line(f"{case:<44} {out:<8} {a:10.3e} {r:10.3e} {f:10.3e}  {tol}")
