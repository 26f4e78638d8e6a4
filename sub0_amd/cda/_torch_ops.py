"""torch.ops namespaces of the MI355X CDA kernels, from the native library.

``libcda_hip_torch.so`` (built from ``sub0_amd/csrc/torch_ops.cpp``) defines
the ops in C++ with ``TORCH_LIBRARY`` over the C ABI of ``libcda_hip.so``:
schemas with ``Tensor(a!)`` on the outputs written in place, CUDA (= HIP)
kernels with ``TORCH_CHECK`` errors (TypeError for dtypes, ValueError for
shapes, NotImplementedError for features the kernels lack), and Meta kernels
so the ops trace under ``torch.compile`` / FakeTensor.  This module loads it
once with ``torch.ops.load_library``, as the reference loads its prebuilt
extensions (``cda/_prebuilt_loader.py:69-80``); C++ callers can load the same
file themselves.

``torch.ops.cda_hip`` -- the product entry points the reference reaches
through its pybind modules (``cda/kernels_cuda/wrappers.py:115-124,
153-156``, ``fa2_cda.py:51-52, 85-95, 166-181``): ``decode``, ``encode``,
``decode_uniform_qk``, ``qk_scores_uniform4``, ``prefill``, ``prefill_hybrid``,
``paged_to_dense``, ``varlen_fwd_hadamard``, ``varlen_fwd``, ``hadamard128``.
``load_pybind_module`` routes its module functions through these ops.

``torch.ops._cda_vllm_fa2_fork_C`` -- the comparator namespace of the
reference's vLLM FA2 fork (``cda/kernels_vllm_fa2_fork/interface.py:
138-162, 234-257, 304-328, 434-461``), with the reference's positional
signatures.  They run in the rotated frame (no Hadamard), fp16, head_dim
128, GQA 4 or 8, and return ``[out, softmax_lse]`` with an empty
``softmax_lse`` (the fork fills it only for ``return_softmax`` with dropout,
which inference never uses); dropout, ALiBi, sliding windows, soft-capping,
split-KV and left padding raise ``NotImplementedError``.
"""
from __future__ import annotations

import os
import threading
from pathlib import Path

import torch

from sub0_amd import _native

NAMESPACES = ("cda_hip", "_cda_vllm_fa2_fork_C")

# SUB0_AMD_TORCH_LIB may name another build of the same library.
TORCH_LIB_PATH = Path(os.environ.get("SUB0_AMD_TORCH_LIB") or
                      Path(_native.__file__).resolve().parent / "_lib" / "libcda_hip_torch.so")

_lock = threading.Lock()
_loaded = False


def load() -> None:
    """Load libcda_hip_torch.so once (after libcda_hip.so, whose soname it
    links against, so both use the same kernel library)."""
    global _loaded
    if _loaded:
        return
    with _lock:
        if _loaded:
            return
        _native.lib()
        if not TORCH_LIB_PATH.is_file():
            raise _native.NativeMissing(
                f"{TORCH_LIB_PATH} not found; build it with `python -m sub0_amd.build`")
        torch.ops.load_library(str(TORCH_LIB_PATH))
        _loaded = True


load()
