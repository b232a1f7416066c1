"""Delta-rule forwards: seeded inputs, canonical Program builders and stage programs."""
from .deltanet import DELTANET_OUTPUTS, build_deltanet_program, make_inputs
from .fused_stages import (build_kkt_fused_program, build_scan_fused_program,
                           build_scan_staged_program, make_kkt_inputs, make_scan_inputs)
from .gdn import (GDN_PROGRAM_INPUTS, build_gdn_program, make_gdn_inputs,
                  prepare_gdn_bindings)
from .inputs import as_oracle_inputs, make_delta_inputs
from .kda import KDA_PROGRAM_INPUTS, build_kda_program, make_kda_inputs, prepare_kda_bindings

__all__ = ["make_delta_inputs", "as_oracle_inputs",
           "build_deltanet_program", "make_inputs", "DELTANET_OUTPUTS",
           "build_gdn_program", "prepare_gdn_bindings", "make_gdn_inputs",
           "GDN_PROGRAM_INPUTS",
           "build_kda_program", "prepare_kda_bindings", "make_kda_inputs", "KDA_PROGRAM_INPUTS",
           "make_scan_inputs", "build_scan_fused_program", "build_scan_staged_program",
           "make_kkt_inputs", "build_kkt_fused_program"]
