"""vLLM general-plugin entry (drop-in for ``cda/vllm_plugin.py``).

vLLM runs every enabled general plugin in each worker process; this one puts
the CDA backend into that process's ``AttentionBackendEnum``.  Declare it in
the installing package's metadata as the entry point
``vllm.general_plugins: cda_v2 = sub0_amd.cda.vllm_plugin:register_cda_v2``
and enable it with ``VLLM_PLUGINS=cda_v2``.
"""
from __future__ import annotations

import os


def register_cda_v2() -> None:
    """Register the backend under the ``CDA`` slot (``vllm_plugin.py:16-30``);
    with ``CDA_V2_ENABLE_MEMORY_SAVING=1`` also size vLLM's pages for
    144-byte slots."""
    from sub0_amd.cda.kernels_cuda.vllm_integration.cda_attn_v2 import (
        enable_cda_memory_saving,
        register_backend,
    )
    if os.environ.get("CDA_V2_ENABLE_MEMORY_SAVING") == "1":
        enable_cda_memory_saving()
    register_backend("CDA")
