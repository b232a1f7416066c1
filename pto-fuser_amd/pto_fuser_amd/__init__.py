"""pto_fuser_amd — MI355X (gfx950) backend for pto-fuser's chunked delta-rule forward.

Direct operators over the C ABI (``ops``: the fused GDN/DeltaNet forward, kkt + inverse, the
tri-inverse and the stage kernels) and the reference's compile stack rebuilt over them: the
Program IR, staged and HIP-graph executors, opaque and fused-kernel registries, gates, cost model,
policy, transforms, templates and ``compile_program``.
"""
from . import _hip
from .compile import CompileResult, compile_program
from .cost import CostModel, Features, Prediction
from .dataflow import Dataflow, ProgramEdit
from .executor import StagedExecutor
from .fused import (FusedContract, FusedKernel, FusedKernelRegistry, default_fused_registry,
                    shared_fused_registry)
from .fusion import FusionDecision, decide, format_decisions as format_fusion_decisions
from .gate import GateResult, frob_rel, gate_determinism, gate_frob_rel, gate_outputs
from .graph import CaptureExecutor, GraphReplayExecutor
from .ir import (EinsumNode, FusedNode, Node, OpaqueNode, Program, TensorOp, TensorRef,
                 VecGlueNode)
from .ops import (chunk_scan, gated_qk, gdn_chunk_forward, kda_chunk_forward, kkt_inverse,
                  qkv_flash, tri_inv)
from .policy import PlannedTransform, Policy
from .registry import OpaqueContract, OpaqueRegistry, capture_mode, default_registry
from .report import CompilationReport, TransformRecord
from .template import (EpilogueUnit, FuseChunkOFlash, FuseContractionEpilogue,
                       FusePerDimChunkOFlash, ScoreTemplate, Template, default_templates,
                       epilogue_report, extract_epilogue_unit)
from .transform import (EnableDirectReads, EnableFusedStore, Transform, TransformResult,
                        canonicalize)

__all__ = [
    "gdn_chunk_forward", "kda_chunk_forward", "kkt_inverse", "tri_inv", "gated_qk", "qkv_flash",
    "chunk_scan",
    "TensorRef", "Node", "EinsumNode", "OpaqueNode", "VecGlueNode", "TensorOp", "FusedNode",
    "Program", "Dataflow", "ProgramEdit", "StagedExecutor", "OpaqueRegistry", "OpaqueContract",
    "default_registry", "capture_mode", "GateResult", "FusedContract", "FusedKernel",
    "FusedKernelRegistry", "default_fused_registry", "shared_fused_registry", "frob_rel",
    "gate_frob_rel", "gate_outputs", "gate_determinism", "CaptureExecutor",
    "GraphReplayExecutor", "FusionDecision", "decide", "format_fusion_decisions", "Transform",
    "TransformResult", "canonicalize", "EnableDirectReads", "EnableFusedStore", "CostModel",
    "Features", "Prediction", "Policy", "PlannedTransform", "CompilationReport",
    "TransformRecord", "CompileResult", "compile_program", "EpilogueUnit",
    "extract_epilogue_unit", "ScoreTemplate", "Template", "default_templates", "FuseContractionEpilogue",
    "FuseChunkOFlash", "FusePerDimChunkOFlash", "epilogue_report",
]
