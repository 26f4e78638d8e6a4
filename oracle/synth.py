"""Deterministic synthetic inputs for the CDA checker (test infrastructure).

This module is part of ``oracle/``: only ``tests/``, ``__graft_entry__.smoke()``
and ``bench.py``'s CPU-baseline leg may import it.

The reference benchmarks draw K/V/Q from ``torch.randn`` under
``torch.manual_seed(0xCDA + N + 97*B)``
(``benchmarks/bench_compute_path_iso_cuda_graph.py:87-100``).  A torch RNG
stream is not guaranteed to be bit-stable across machines and versions, and
the golden fixtures must regenerate their inputs bit-for-bit on the GPU box,
so this generator uses only integer arithmetic plus one correctly rounded
float64 division and the correctly rounded float64->float16 cast:

* splitmix64 produces 64-bit words;
* four 16-bit uniforms are summed (Irwin-Hall, n=4), giving an integer with
  mean 4*(2^16-1)/2 and variance 4*(2^32-1)/12;
* the centred integer is divided by the standard deviation in float64 and
  rounded to float16.

The result is approximately N(0, 1) (bounded at about +-3.46 sigma), which is
what the configs ask for.  "Outlier channels" follow BASELINE config 0: K has
``n_outliers`` seeded channels scaled by 8 (the channel set is drawn from the
same stream).
"""
from __future__ import annotations

import numpy as np

_MASK64 = np.uint64(0xFFFFFFFFFFFFFFFF)
_GOLDEN = np.uint64(0x9E3779B97F4A7C15)


def _splitmix64(seed: int, n: int) -> np.ndarray:
    """n successive splitmix64 outputs for a stream started at ``seed``."""
    with np.errstate(over="ignore"):
        idx = np.arange(1, n + 1, dtype=np.uint64)
        z = (np.uint64(seed & 0xFFFFFFFFFFFFFFFF) + idx * _GOLDEN) & _MASK64
        z = ((z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)) & _MASK64
        z = ((z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)) & _MASK64
        z = z ^ (z >> np.uint64(31))
    return z


_IH_MEAN = 4 * 65535 / 2.0
_IH_STD = float(np.sqrt(4 * (65536.0 ** 2 - 1) / 12.0))


def normal_f16(seed: int, shape) -> np.ndarray:
    """Approximately standard-normal float16 array, bit-reproducible."""
    n = int(np.prod(shape)) if len(shape) else 1
    w = _splitmix64(seed, n)
    s = ((w & np.uint64(0xFFFF)) + ((w >> np.uint64(16)) & np.uint64(0xFFFF))
         + ((w >> np.uint64(32)) & np.uint64(0xFFFF)) + (w >> np.uint64(48)))
    x = (s.astype(np.float64) - _IH_MEAN) / _IH_STD
    return x.astype(np.float16).reshape(shape)


def outlier_channels(seed: int, d: int = 128, n_outliers: int = 4) -> np.ndarray:
    """Sorted distinct channel ids in [0, d) chosen by the seeded stream."""
    w = _splitmix64(seed ^ 0x5EED, 4 * d)
    chosen: list[int] = []
    for v in w:
        c = int(v % np.uint64(d))
        if c not in chosen:
            chosen.append(c)
        if len(chosen) == n_outliers:
            break
    return np.array(sorted(chosen), dtype=np.int64)


def kv_with_outliers(seed: int, shape, *, n_outliers: int = 4, factor: float = 8.0):
    """float16 K-like data: N(0,1) with ``n_outliers`` channels scaled by ``factor``.

    The scaling happens in float32 and is rounded once to float16 (an exact
    multiply for a power-of-two factor).
    """
    x = normal_f16(seed, shape)
    if n_outliers:
        ch = outlier_channels(seed, shape[-1], n_outliers)
        xf = x.astype(np.float32)
        xf[..., ch] *= np.float32(factor)
        x = xf.astype(np.float16)
    return x


def permuted_block_table(seed: int, B: int, blocks_per_seq: int) -> np.ndarray:
    """(B, blocks_per_seq) int32: a seeded permutation of B*blocks_per_seq pages."""
    n = B * blocks_per_seq
    keys = _splitmix64(seed ^ 0xB10C, n)
    perm = np.argsort(keys, kind="stable").astype(np.int32)
    return perm.reshape(B, blocks_per_seq)


def cfg_seed(B: int, N: int) -> int:
    """The reference's per-cell seed convention ``0xCDA + N + 97*B``."""
    return 0xCDA + N + 97 * B
