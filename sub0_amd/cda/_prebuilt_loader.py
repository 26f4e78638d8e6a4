"""Loader for the MI355X CDA kernels (drop-in for ``cda/_prebuilt_loader.py``).

The reference resolves each logical kernel name to a prebuilt CUDA ``.so``
(``cda/_prebuilt_loader.py:56-80``).  Here every name resolves to one HIP
library, ``sub0_amd/_lib/libcda_hip.so``, reached through its C ABI.
``load_pybind_module(name)`` returns a module object whose attributes have
the reference's positional signatures and call the ``torch.ops.cda_hip``
ops; ``load_torch_ops_library(name)`` loads the native ``TORCH_LIBRARY`` build,
``sub0_amd/_lib/libcda_hip_torch.so``, with ``torch.ops.load_library`` and
returns the namespace (``cda_hip``, or the FA2-fork comparator namespace
``_cda_vllm_fa2_fork_C``; see :mod:`sub0_amd.cda._torch_ops`).  Both are
``lru_cache``d and idempotent, and raise :class:`PrebuiltMissing` (an ``ImportError``) when the artefact is
missing or the name is not provided, as the reference does
(``_prebuilt_loader.py:41-53``).
"""
from __future__ import annotations

import math
import sys
from functools import lru_cache
from types import ModuleType

import torch

from sub0_amd import _native

_DECODE_NAMES = {
    "_v1_decode_hmma_k4v4_gs4": (4, False),
    "_v1_decode_hmma_k4v4_gs8": (8, False),
    "_v1_decode_hmma_k4v2_gs4": (4, True),
    "_v1_decode_hmma_k4v2_gs8": (8, True),
}


class PrebuiltMissing(ImportError):
    """Raised when no artefact matches the requested logical name."""


def _lib_or_raise():
    try:
        return _native.lib()
    except _native.NativeMissing as e:
        raise PrebuiltMissing(str(e)) from e


def _flat_cache(kv_cache: torch.Tensor) -> torch.Tensor:
    """Accept (num_slots, H_kv, slot_w) or vLLM's (num_blocks, bs, H_kv, slot_w)."""
    if kv_cache.dim() == 4:
        nb, bs, h, w = kv_cache.shape
        return kv_cache.view(nb * bs, h, w)
    return kv_cache


def _make_decode_module(name: str, gs: int, k4v2: bool) -> ModuleType:
    mod = ModuleType(name)
    mod.__doc__ = ("CDA split-K decode (%s, group size %d) on MI355X; replaces the "
                   "reference's %s.so." % ("K4V2, 104-byte slots" if k4v2 else "K4V4", gs, name))

    def cda_decode_full_hmma_v3(Q, kv_cache, block_table, seq_lens, cb_K, cb_V,
                                rotation_fp32, rotation_fp16, out, group_size, block_size,
                                tile_N, max_seq_len, scale):
        """Positional signature of the reference call (wrappers.py:115-124)."""
        if int(group_size) != gs:
            raise ValueError(f"{name} is built for group_size={gs}, got {group_size}")
        if k4v2 and (cb_K.numel(), cb_V.numel()) != (16, 4):
            raise ValueError(f"{name} reads K4V2 caches: cb_K needs 16 levels, cb_V 4")
        torch.ops.cda_hip.decode(
            Q, _flat_cache(kv_cache), block_table, seq_lens, cb_K, cb_V, rotation_fp32,
            rotation_fp16 if rotation_fp16 is not None else rotation_fp32, out, gs,
            int(block_size), int(tile_N), int(max_seq_len),
            float(scale) if scale is not None else 1.0 / math.sqrt(Q.shape[-1]))

    mod.cda_decode_full_hmma_v3 = cda_decode_full_hmma_v3
    return mod


def _make_encode_module(name: str) -> ModuleType:
    mod = ModuleType(name)
    mod.__doc__ = ("CDA fused paged encode on MI355X: K4V4 and K2V2 slots, or the legacy "
                   "K4V2 slot when cb_V has 4 levels and cb_K 16.")

    def cda_paged_encode_fused(K, V, slot_mapping, flat_cache, cb_K, cb_V):
        """Positional signature of the reference call (wrappers.py:153-156)."""
        torch.ops.cda_hip.encode(K, V, slot_mapping, _flat_cache(flat_cache), cb_K, cb_V)

    mod.cda_paged_encode_fused = cda_paged_encode_fused
    return mod


def _register_ops():
    """Load libcda_hip_torch.so (torch.ops.cda_hip and the fork namespace)."""
    try:
        from sub0_amd.cda import _torch_ops
        _torch_ops.load()
    except _native.NativeMissing as e:
        raise PrebuiltMissing(str(e)) from e


def _factories():
    f = {n: (lambda n=n, g=g: _make_decode_module(n, *g)) for n, g in _DECODE_NAMES.items()}
    # The kv-update modules (hmma_loader.py:40-43) have no caller in the
    # reference that shows their symbol; they carry the fused encode.
    for n in ("_v1_paged_encode_fused", "_v1_kv_update_k4v4", "_v1_kv_update_k4v2"):
        f[n] = lambda n=n: _make_encode_module(n)
    try:
        from sub0_amd.cda.kernels_cuda import _prefill_modules
    except ImportError:
        _prefill_modules = None
    if _prefill_modules is not None:
        f.update(_prefill_modules.FACTORIES)
    return f


@lru_cache(maxsize=64)
def load_pybind_module(name: str) -> ModuleType:
    """Return the module object for logical kernel ``name``."""
    fac = _factories().get(name)
    if fac is None:
        raise PrebuiltMissing(
            f"Kernel module '{name}' is not provided by the MI355X build "
            f"(available: {sorted(_factories())}).")
    _lib_or_raise()
    _register_ops()
    module = fac()
    sys.modules[name] = module
    return module


@lru_cache(maxsize=64)
def load_torch_ops_library(name: str):
    """TORCH_LIBRARY flavour (reference ``_prebuilt_loader.py:69-80``): the
    torch.ops namespace ``name`` once its ops are registered."""
    namespaces = ("cda_hip", "_cda_vllm_fa2_fork_C")
    if name not in namespaces:
        raise PrebuiltMissing(
            f"torch.ops library '{name}' is not provided by the MI355X build "
            f"(available: {list(namespaces)}).")
    _lib_or_raise()
    _register_ops()
    return getattr(torch.ops, name)
