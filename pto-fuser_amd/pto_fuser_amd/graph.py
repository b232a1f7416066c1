"""Graph-replay backend: a whole Program captured into one HIP graph (src/pto_fuser/graph.py).

``GraphReplayExecutor.capture`` runs the program eagerly a few times on a side stream (first-call
library setup — hipBLASLt heuristics, the HIP library load — happens there, outside the graph),
then records one run into a ``torch.cuda.CUDAGraph`` (a hipGraph on ROCm) over static input
buffers.  ``replay`` copies new operands into those buffers and launches the graph: the program's
tens to hundreds of kernel launches become one graph launch.

Everything the program launches is capturable as it stands: the HIP stage kernels enqueue on the
current stream and allocate nothing, the opaque tri-inverse needs no host synchronisation (it
launches on the current stream, unlike the reference's raw launch), and torch's own kernels
allocate from the graph's private pool.  Shapes are fixed at capture time.
"""
from __future__ import annotations

from typing import Dict, Optional

import torch

from . import registry as _registry
from .executor import StagedExecutor, _cast, library_modes
from .fused import FusedKernelRegistry
from .ir import EinsumNode, Program
from .registry import OpaqueRegistry

__all__ = ["CaptureExecutor", "GraphReplayExecutor"]


class CaptureExecutor(StagedExecutor):
    """A StagedExecutor whose contractions go through per-node runners built once (with the
    node's read-mode / fused-store annotations fixed at build time), so the captured region is
    launches only."""

    def __init__(self, registry: Optional[OpaqueRegistry] = None,
                 fused: Optional[FusedKernelRegistry] = None) -> None:
        super().__init__(registry, fused=fused)
        self._runners: Dict[tuple, object] = {}

    def _exec(self, node, env):
        if isinstance(node, EinsumNode):
            a, b = (env[n] for n in node.inputs)
            return _cast(self._runner(node, a, b)(a, b), node.out_dtype)
        return super()._exec(node, env)

    def _runner(self, node: EinsumNode, a: torch.Tensor, b: torch.Tensor):
        key = (node.equation, tuple(a.shape), tuple(b.shape), a.dtype, b.dtype,
               node.read_mode, node.fuse_out)
        runner = self._runners.get(key)
        if runner is None:
            eq, mode, fuse, core = node.equation, node.read_mode, node.fuse_out, self.einsum

            def runner(x, y, eq=eq, mode=mode, fuse=fuse, core=core):
                with library_modes(mode, fuse):
                    return core(eq, x, y)
            self._runners[key] = runner
        return runner


class GraphReplayExecutor:
    """Capture a Program into one HIP graph; replay it as a single launch."""

    def __init__(self, registry: Optional[OpaqueRegistry] = None,
                 fused: Optional[FusedKernelRegistry] = None) -> None:
        self._exec = CaptureExecutor(registry, fused)
        self._graph: Optional[torch.cuda.CUDAGraph] = None
        self._static_in: Dict[str, torch.Tensor] = {}
        self._out: Dict[str, torch.Tensor] = {}
        self.program: Optional[Program] = None

    def capture(self, program: Program, bindings: Dict[str, torch.Tensor],
                warmup: int = 3) -> "GraphReplayExecutor":
        missing = [n for n in program.inputs if n not in bindings]
        if missing:
            raise ValueError(f"missing bindings for inputs: {missing}")
        self._static_in = {k: bindings[k].clone() for k in program.inputs}
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(max(1, warmup)):
                self._exec.run(program, self._static_in, return_env=True)
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()

        graph = torch.cuda.CUDAGraph()
        # captured on the warmup stream: the fused kernels' workspaces are cached per stream
        # and were allocated there by the warmup (capture itself must not allocate them)
        with torch.cuda.graph(graph, stream=side):
            with _registry.capture_mode():
                env = self._exec.run(program, self._static_in, return_env=True)
        torch.cuda.synchronize()
        self._graph = graph
        self.program = program
        self._out = {name: env[name] for name in program.outputs}
        return self

    def replay(self, bindings: Dict[str, torch.Tensor],
               clone: bool = True) -> Dict[str, torch.Tensor]:
        """Replay on ``bindings`` (the captured shapes).  The outputs live in the graph's pool;
        ``clone=True`` returns copies that survive the next replay."""
        if self._graph is None:
            raise RuntimeError("capture() must be called before replay()")
        for name, buf in self._static_in.items():
            src = bindings[name]
            if tuple(src.shape) != tuple(buf.shape):
                raise ValueError(f"replay shape {tuple(src.shape)} for {name!r} != captured "
                                 f"{tuple(buf.shape)} (a new shape needs a new capture)")
            buf.copy_(src)
        self._graph.replay()
        if clone:
            return {k: v.clone() for k, v in self._out.items()}
        return dict(self._out)
