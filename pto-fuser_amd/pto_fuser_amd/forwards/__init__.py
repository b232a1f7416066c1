"""Delta-rule forwards: inputs, Program builders and stage programs."""
from .inputs import as_oracle_inputs, make_delta_inputs

__all__ = ["make_delta_inputs", "as_oracle_inputs"]
