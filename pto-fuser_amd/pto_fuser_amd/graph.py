"""Graph replay: a whole Program recorded once as a HIP graph and replayed as one launch.

The reference records its programs with NPU graphs (src/pto_fuser/graph.py:80-138); here the
recording is a ``torch.cuda.CUDAGraph``, which is a hipGraph on ROCm.  ``capture``:

1. copies the bindings into static input buffers (replays read from them);
2. runs the program eagerly ``warmup`` times on a private stream — first-call work (the HIP
   library load, GEMM heuristics, the fused kernels' per-stream workspaces) happens there;
3. records one run on that same stream, inside ``capture_mode()``.

``replay`` copies new operands of the captured shapes into the static buffers and launches the
graph.  Every node of a program is capturable as it stands: the HIP kernels enqueue on the
current stream and allocate nothing, and torch's kernels allocate from the graph's private pool.
"""
from __future__ import annotations

from typing import Dict, Optional

import torch

from .executor import StagedExecutor
from .fused import FusedKernelRegistry
from .ir import Program
from .registry import OpaqueRegistry, capture_mode

__all__ = ["CaptureExecutor", "GraphReplayExecutor"]


class CaptureExecutor(StagedExecutor):
    """The staged executor as used for recording: every step runs inside ``capture_mode()``."""

    def run(self, program: Program, bindings: Dict[str, torch.Tensor], return_env: bool = False):
        with capture_mode():
            return super().run(program, bindings, return_env)


class GraphReplayExecutor:
    def __init__(self, registry: Optional[OpaqueRegistry] = None,
                 fused: Optional[FusedKernelRegistry] = None) -> None:
        self._eager = StagedExecutor(registry, fused=fused)
        self._recorder = CaptureExecutor(registry, fused=fused)
        self._graph: Optional[torch.cuda.CUDAGraph] = None
        self._inputs: Dict[str, torch.Tensor] = {}
        self._outputs: Dict[str, torch.Tensor] = {}
        self.program: Optional[Program] = None

    def capture(self, program: Program, bindings: Dict[str, torch.Tensor],
                warmup: int = 3) -> "GraphReplayExecutor":
        absent = [n for n in program.inputs if n not in bindings]
        if absent:
            raise ValueError(f"missing bindings for program inputs: {absent}")
        self._inputs = {n: bindings[n].clone() for n in program.inputs}
        stream = torch.cuda.Stream()
        stream.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(stream):
            for _ in range(max(1, warmup)):
                self._eager.run(program, self._inputs)
        stream.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            env = self._recorder.run(program, self._inputs, return_env=True)
        torch.cuda.synchronize()
        self._graph, self.program = graph, program
        self._outputs = {n: env[n] for n in program.outputs}
        return self

    def replay(self, bindings: Dict[str, torch.Tensor],
               clone: bool = True) -> Dict[str, torch.Tensor]:
        """Launch the graph on ``bindings`` (the captured shapes).  The outputs live in the
        graph's pool and are overwritten by the next replay; ``clone=True`` returns copies."""
        if self._graph is None:
            raise RuntimeError("replay() needs a graph: call capture() first")
        for name, buf in self._inputs.items():
            src = bindings[name]
            if src.shape != buf.shape:
                raise ValueError(f"{name!r} has shape {tuple(src.shape)} but the graph was "
                                 f"captured for {tuple(buf.shape)}; capture again for a new shape")
            buf.copy_(src)
        self._graph.replay()
        return {n: (t.clone() if clone else t) for n, t in self._outputs.items()}
