"""Module-level handles on the four backend classes, so that vLLM's registry
can resolve them by dotted path (``cda/vllm_integration/_backend_eager.py``).

The classes are built by
:func:`sub0_amd.cda.kernels_cuda.vllm_integration.cda_attn_v2.get_backend_classes`;
importing this module builds them (with vLLM's base classes when vLLM is
importable, with plain stand-ins otherwise).
"""
from sub0_amd.cda.kernels_cuda.vllm_integration.cda_attn_v2 import get_backend_classes

(
    CDAv2AttentionBackend,
    CDAv2AttentionImpl,
    CDAv2AttentionMetadataBuilder,
    CDAv2AttentionMetadata,
) = get_backend_classes()

__all__ = [
    "CDAv2AttentionBackend",
    "CDAv2AttentionImpl",
    "CDAv2AttentionMetadataBuilder",
    "CDAv2AttentionMetadata",
]
