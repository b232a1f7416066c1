"""CPU baseline of the GDN chunked forward — TEST INFRASTRUCTURE (bench.py's cpu_baseline leg).

Times the fp32 numpy oracle (``gdn_oracle.gdn_reference`` in the reference's per-(b, h, chunk)
loop order, restating examples/attention/_gdn_full.py:57-97) on the host's cores, over the same
seeded inputs the GPU run uses.  The (b, h) chains are independent, so a pool of worker
processes splits them; each worker runs its chains with one BLAS thread.  A one-process figure
over a subset of chains (scaled to the whole workload in B*H) is reported beside it.

bench.py runs this as a child process before it touches the GPU, and reads the one JSON line
it prints::

    python -m oracle.cpu_baseline --B 4 --H 16 --T 4096 --workers 16 --runs 5
"""
from __future__ import annotations

import argparse
import json
import multiprocessing as mp
import os
import statistics
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "pto-fuser_amd"))
sys.path.insert(0, ROOT)

from oracle.gdn_oracle import gdn_reference  # noqa: E402

_X = {}          # the workload, set before the pool forks (copy-on-write in the workers)


def _chains(idx):
    """Run the oracle over the chains listed in ``idx`` (flat b*H + h indices)."""
    from threadpoolctl import threadpool_limits
    B, H = _X["q"].shape[:2]
    with threadpool_limits(1):
        for i in idx:
            b, h = divmod(i, H)
            sl = (slice(b, b + 1), slice(h, h + 1))
            gdn_reference(_X["q"][sl], _X["k"][sl], _X["v"][sl], _X["beta"][sl], _X["g"][sl],
                          C=_X["C"], dtype=np.float32, loop=True)
    return len(idx)


def measure(B: int, H: int, T: int, C: int = 64, workers: int = 0, runs: int = 5,
            single_chains: int = 8, seed: int = 0) -> dict:
    from pto_fuser_amd.forwards.inputs import make_delta_inputs
    import torch

    inp = make_delta_inputs(B, H, T, kind="gdn", dtype=torch.bfloat16, seed=seed)
    for n in ("q", "k", "v", "beta", "g"):
        _X[n] = inp[n].float().numpy()
    _X["C"] = C
    n_chains = B * H
    host = os.cpu_count() or 1
    share = int(os.environ.get("OMP_NUM_THREADS", host))
    workers = workers or max(1, min(host, share, n_chains))
    groups = [list(range(w, n_chains, workers)) for w in range(workers)]

    # one process, a subset of the chains, scaled to the whole workload
    _chains([0])
    sub = list(range(min(single_chains, n_chains)))
    t0 = time.perf_counter()
    _chains(sub)
    t_one = (time.perf_counter() - t0) * n_chains / len(sub)

    ctx = mp.get_context("fork")
    times = []
    with ctx.Pool(workers) as pool:
        pool.map(_chains, [[g[0]] for g in groups])          # warm every worker
        for _ in range(runs):
            t0 = time.perf_counter()
            assert sum(pool.map(_chains, groups)) == n_chains
            times.append(time.perf_counter() - t0)
    t = statistics.median(times)
    return {
        "value": B * T / t, "unit": "tokens/s", "cores": workers, "kind": "port",
        "host_cpus": host, "cpu_share": share,
        "single_core_value": B * T / t_one,
        "sample": (f"whole workload B{B} H{H} T{T} ({n_chains} chains x {T // C} chunks), fp32 "
                   f"numpy oracle in the reference's b,h,c loop order, chains split over "
                   f"{workers} worker processes (1 BLAS thread each; host has {host} CPUs, "
                   f"share {share}), median of {runs} runs "
                   f"({', '.join(f'{s:.3f}' for s in times)} s); single_core_value: one process "
                   f"over {len(sub)} chains ({t_one * len(sub) / n_chains:.2f} s), scaled by "
                   f"{n_chains}/{len(sub)}"),
    }


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description="CPU baseline of the GDN chunked forward")
    ap.add_argument("--B", type=int, default=4)
    ap.add_argument("--H", type=int, default=16)
    ap.add_argument("--T", type=int, default=4096)
    ap.add_argument("--C", type=int, default=64)
    ap.add_argument("--workers", type=int, default=0, help="0: the host's CPU share")
    ap.add_argument("--runs", type=int, default=5)
    args = ap.parse_args(argv)
    print(json.dumps(measure(args.B, args.H, args.T, args.C, args.workers, args.runs)), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
