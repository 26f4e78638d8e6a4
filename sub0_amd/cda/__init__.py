"""cda -- drop-in mirror of the reference package surface on MI355X.

Reference: ``cda/__init__.py``.  The kernels behind it are the HIP kernels of
``sub0_amd/csrc`` reached through ``cda._prebuilt_loader``.
"""
__version__ = "0.1.0.mi355x"
