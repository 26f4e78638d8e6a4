"""Module objects for the prefill kernel names of the reference loader
(``hmma_loader.py:45-58``): the paged -> dense rotated loader, the fused
varlen forward with the Hadamard prologue/epilogue, and the Hadamard-128
helper.  Each calls the ``torch.ops.cda_hip`` op that wraps the MI355X C ABI.
"""
from __future__ import annotations

from types import ModuleType

import torch


def _flat_cache(kv_cache):
    if kv_cache.dim() == 4:
        nb, bs, h, w = kv_cache.shape
        return kv_cache.view(nb * bs, h, w)
    return kv_cache


def _loader_module(name: str) -> ModuleType:
    mod = ModuleType(name)
    mod.__doc__ = ("Paged K4V4 (or, with a 4-level cb_V, the legacy K4V2) cache -> dense "
                   "rotated fp16 K/V (MI355X).")

    def cda_fa2_paged_cache_to_dense_rotated(kv_cache, block_table, seq_lens, cb_K, cb_V,
                                             block_size, max_seq_len):
        """Positional signature of the reference call (fa2_cda.py:85-95)."""
        return torch.ops.cda_hip.paged_to_dense(_flat_cache(kv_cache), block_table, seq_lens,
                                                cb_K, cb_V, int(block_size), int(max_seq_len))

    mod.cda_fa2_paged_cache_to_dense_rotated = cda_fa2_paged_cache_to_dense_rotated
    return mod


def _varlen_module(name: str) -> ModuleType:
    mod = ModuleType(name)
    mod.__doc__ = "Causal varlen attention with Hadamard prologue/epilogue (MI355X)."

    def cda_fa2_varlen_fwd_hadamard(Q, k_rot, v_rot, out, cu_q, cu_k, seqused_k, max_q, max_k,
                                    scale):
        """Positional signature of the reference call (fa2_cda.py:166-181)."""
        torch.ops.cda_hip.varlen_fwd_hadamard(Q, k_rot, v_rot, out, cu_q, cu_k, seqused_k,
                                              int(max_q), int(max_k), float(scale))

    mod.cda_fa2_varlen_fwd_hadamard = cda_fa2_varlen_fwd_hadamard
    return mod


def _hadamard_module(name: str) -> ModuleType:
    mod = ModuleType(name)
    mod.__doc__ = "Row-wise Hadamard-128 transform of fp16 rows (MI355X)."

    def hadamard128_fp16(x, y, scale):
        """Positional signature of the reference call (fa2_cda.py:51-52)."""
        torch.ops.cda_hip.hadamard128(x, y, float(scale))

    mod.hadamard128_fp16 = hadamard128_fp16
    return mod


FACTORIES = {
    "_v1_fa2_cda_loader_k4v4": lambda: _loader_module("_v1_fa2_cda_loader_k4v4"),
    "_v1_fa2_cda_loader_k4v2": lambda: _loader_module("_v1_fa2_cda_loader_k4v2"),
    "_v1_fa2_cda_varlen_fused": lambda: _varlen_module("_v1_fa2_cda_varlen_fused"),
    "_v1_fa2_cda_hadamard128": lambda: _hadamard_module("_v1_fa2_cda_hadamard128"),
}
