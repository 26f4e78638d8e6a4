"""Logical-kernel loaders (drop-in for ``cda/kernels_cuda/hmma_loader.py``).

Same names and argument checks as the reference (``hmma_loader.py:27-59``);
each resolves through :func:`sub0_amd.cda._prebuilt_loader.load_pybind_module`
to the MI355X HIP library, including the K4V2 names (decode, kv update and
dense loader of the legacy 104-byte slot).
"""
from __future__ import annotations

from functools import lru_cache

from sub0_amd.cda._prebuilt_loader import load_pybind_module


@lru_cache(maxsize=8)
def load_decode_hmma(k4v2: bool = False, group_size: int = 4):
    if group_size not in (4, 8):
        raise ValueError(f"group_size must be 4 or 8 (got {group_size})")
    v_tag = "k4v2" if k4v2 else "k4v4"
    return load_pybind_module(f"_v1_decode_hmma_{v_tag}_gs{group_size}")


@lru_cache(maxsize=2)
def load_paged_encode_fused():
    return load_pybind_module("_v1_paged_encode_fused")


@lru_cache(maxsize=4)
def load_kv_cache_update(k4v2: bool = False):
    name = "_v1_kv_update_k4v2" if k4v2 else "_v1_kv_update_k4v4"
    return load_pybind_module(name)


@lru_cache(maxsize=4)
def load_fa2_cda_loader(k4v2: bool = False):
    name = "_v1_fa2_cda_loader_k4v2" if k4v2 else "_v1_fa2_cda_loader_k4v4"
    return load_pybind_module(name)


@lru_cache(maxsize=1)
def load_fa2_cda_hadamard():
    return load_pybind_module("_v1_fa2_cda_hadamard128")


@lru_cache(maxsize=1)
def load_fa2_cda_varlen_fused():
    return load_pybind_module("_v1_fa2_cda_varlen_fused")


__all__ = [
    "load_decode_hmma",
    "load_paged_encode_fused",
    "load_kv_cache_update",
    "load_fa2_cda_loader",
    "load_fa2_cda_hadamard",
    "load_fa2_cda_varlen_fused",
]
