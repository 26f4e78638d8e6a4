"""sub0_amd -- Compressed-Domain Attention (CDA) hot path for AMD MI355X (gfx950).

Layout:
  csrc/        hand-written HIP kernels + the C ABI (include/cda_hip.h)
  build.py     hipcc recipe -> _lib/libcda_hip.so
  _native.py   ctypes binding of the C ABI (torch = device memory + streams)
  cda/         drop-in mirror of the reference's Python surface
               (cda._prebuilt_loader, cda.kernels_cuda.*, cda.vllm_plugin, ...)

``install_cda_alias()`` registers ``sub0_amd.cda`` as the top-level ``cda``
package so code written against the reference imports unchanged.
"""
from __future__ import annotations

import sys

__version__ = "0.1.0"


def install_cda_alias() -> None:
    """Make ``import cda`` resolve to ``sub0_amd.cda`` (idempotent)."""
    import importlib
    import pkgutil

    pkg = importlib.import_module("sub0_amd.cda")
    sys.modules.setdefault("cda", pkg)
    for mod in pkgutil.walk_packages(pkg.__path__, prefix="sub0_amd.cda."):
        name = mod.name
        if name.endswith("_backend_eager"):
            continue          # imported on demand (needs the backend classes)
        m = importlib.import_module(name)
        sys.modules.setdefault("cda." + name[len("sub0_amd.cda."):], m)
