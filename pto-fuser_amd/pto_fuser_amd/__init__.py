"""pto_fuser_amd — MI355X (gfx950) backend for pto-fuser's chunked delta-rule forward."""
from . import _hip
from .ops import gdn_chunk_forward, kkt_inverse, tri_inv

__all__ = ["gdn_chunk_forward", "kkt_inverse", "tri_inv"]
