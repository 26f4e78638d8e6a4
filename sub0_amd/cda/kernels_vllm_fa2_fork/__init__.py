"""The FA2-fork comparator namespace (reference ``cda/kernels_vllm_fa2_fork``):
``build.load()`` registers ``torch.ops._cda_vllm_fa2_fork_C``."""

from .interface import (  # noqa: E402
    dequantize_compressed_kv,
    flash_attn_varlen_compressed_kv_func,
    flash_attn_varlen_compressed_kv_fused_func,
    flash_attn_varlen_func,
    register_vllm_backend,
)

__all__ = [
    "dequantize_compressed_kv",
    "flash_attn_varlen_compressed_kv_fused_func",
    "flash_attn_varlen_compressed_kv_func",
    "flash_attn_varlen_func",
    "register_vllm_backend",
]
