"""Loader of the FA2-fork comparator ops (reference
``cda/kernels_vllm_fa2_fork/build.py``): ``load()`` makes sure
``torch.ops._cda_vllm_fa2_fork_C`` is registered; idempotent."""
from __future__ import annotations

from sub0_amd.cda._prebuilt_loader import load_torch_ops_library

EXTENSION_NAME = "_cda_vllm_fa2_fork_C"


def load(*args, **kwargs):
    load_torch_ops_library(EXTENSION_NAME)
