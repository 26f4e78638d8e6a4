"""CDA kernels on MI355X (drop-in for ``cda/kernels_cuda/__init__.py``)."""
from sub0_amd.cda.kernels_cuda.hmma_loader import (
    load_decode_hmma,
    load_fa2_cda_hadamard,
    load_fa2_cda_loader,
    load_fa2_cda_varlen_fused,
    load_kv_cache_update,
    load_paged_encode_fused,
)

__all__ = [
    "load_decode_hmma",
    "load_fa2_cda_hadamard",
    "load_fa2_cda_loader",
    "load_fa2_cda_varlen_fused",
    "load_kv_cache_update",
    "load_paged_encode_fused",
]
