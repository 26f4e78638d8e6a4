"""Codebooks, rotation and slot containers (drop-in for ``cda/algorithm/compression.py``).

The serving path needs the tables, not the pure-torch encode: the
backend takes ``Compressor(...).codebook`` and ``.rotation`` and hands them
to the HIP kernels (reference ``cda_attn_v2.py:309-337``).  This module
builds those tables on the host:

* :func:`hadamard_matrix` -- Sylvester Hadamard / sqrt(d) in fp32
  (reference ``compression.py:43-57``);
* :func:`uniform_centroids` (``:75-83``);
* :func:`lloyd_max_centroids_beta` / :func:`lloyd_max_centroids`
  (``:86-155``): Lloyd-Max on coordinate 0 of unit-normalised Gaussian
  samples.  The steps (torch CPU generator seeded 0xCDA, ``randn``, norm
  clamp 1e-12, nearest-centroid E-step with first-index ties, per-level
  ``mean`` M-step that keeps empty levels, stop when the largest shift is
  below ``tol``, sorted result) must match the reference's to give the same
  fp32 values, so they do; the samples are always drawn on the CPU, which
  makes the table identical on every device.
* :class:`Compressor` -- holds ``rotation``/``codebook`` for one role.  Its
  ``encode``/``decode`` run on the GPU through the HIP encoder (a dense
  variant of the paged encode); there is no CPU path.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from functools import lru_cache
from typing import Optional

import torch
from torch import Tensor


def hadamard_matrix(d: int, *, dtype: torch.dtype = torch.float32,
                    device: torch.device | str | None = None) -> Tensor:
    """Sylvester Hadamard of order ``d`` scaled by 1/sqrt(d) (so H = H^T = H^-1)."""
    if d <= 0 or (d & (d - 1)):
        raise ValueError(f"d must be a positive power of two, got {d}")
    i = torch.arange(d)
    parity = torch.zeros(d, d, dtype=torch.int64)
    bits = i.unsqueeze(1) & i.unsqueeze(0)
    while bool(bits.any()):
        parity ^= bits & 1
        bits = bits >> 1
    sign = 1.0 - 2.0 * parity.to(torch.float32)
    # Same fp32 entry as the reference: fp32(1) / fp32(sqrt(d)).
    h = torch.tensor(1.0, dtype=torch.float32) / torch.tensor(d ** 0.5, dtype=torch.float32)
    return (sign * h).to(dtype=dtype, device=device).contiguous()


def half_rotate_pair(d: int, *, dtype: torch.dtype = torch.float32,
                     device: torch.device | str | None = None) -> Tensor:
    """The rotation applied once to Q, K and V and, inverted, to the output
    (compression.py:60-67): the orthonormal Sylvester Hadamard is its own
    inverse, so one matrix serves both directions."""
    return hadamard_matrix(d, dtype=dtype, device=device)


def uniform_centroids(num_levels: int, *, dtype: torch.dtype = torch.float32,
                      device: torch.device | str | None = None) -> Tensor:
    """Bin midpoints of ``num_levels`` equal bins over [-1, 1]."""
    edges = torch.linspace(-1.0, 1.0, num_levels + 1, dtype=dtype, device=device)
    return ((edges[:-1] + edges[1:]) * 0.5).contiguous()


def lloyd_max_centroids(num_levels: int, samples: Tensor, *, n_iters: int = 50,
                        init: Optional[Tensor] = None, tol: float = 1e-7) -> Tensor:
    """Lloyd-Max iteration on 1-D samples; returns sorted centroids."""
    xs = samples.flatten()
    cb = (uniform_centroids(num_levels, dtype=xs.dtype, device=xs.device)
          if init is None else init).clone()
    for _ in range(n_iters):
        nearest = (xs.unsqueeze(-1) - cb.unsqueeze(0)).pow_(2).argmin(dim=-1)
        updated = cb.clone()
        for level in range(num_levels):
            members = xs[nearest == level]
            if members.numel():
                updated[level] = members.mean()
        shift = float((updated - cb).abs().max())
        cb = updated
        if shift < tol:
            break
    return cb.sort().values.contiguous()


@lru_cache(maxsize=16)
def _lloyd_beta_cpu(num_levels: int, d: int, n_samples: int, n_iters: int, seed: int) -> Tensor:
    gen = torch.Generator(device="cpu").manual_seed(seed)
    x = torch.randn(n_samples, d, dtype=torch.float32, generator=gen)
    unit = x / x.norm(dim=-1, keepdim=True).clamp_min(1e-12)
    return lloyd_max_centroids(num_levels, unit[:, 0], n_iters=n_iters)


def lloyd_max_centroids_beta(num_levels: int, d: int, *, n_samples: int = 100_000,
                             n_iters: int = 50, seed: int = 0xCDA,
                             device: torch.device | str | None = None,
                             dtype: torch.dtype = torch.float32) -> Tensor:
    """Lloyd-Max centroids for one coordinate of a uniform point on S^(d-1).

    Samples are drawn on the CPU generator whatever ``device`` is, then the
    table is moved; the result is cached per (levels, d, n, iters, seed).
    """
    if dtype != torch.float32:
        raise ValueError("lloyd_max_centroids_beta builds fp32 tables")
    cb = _lloyd_beta_cpu(int(num_levels), int(d), int(n_samples), int(n_iters), int(seed))
    return cb.to(device=device).clone()


def pack_4bit(idx: Tensor) -> Tensor:
    """(..., D) codes in [0, 16) -> (..., D/2) bytes, even dim in the high nibble."""
    idx = idx.to(torch.uint8)
    if idx.size(-1) % 2:
        raise ValueError(f"4-bit pack requires even last dim, got {idx.size(-1)}")
    return ((idx[..., 0::2] << 4) | idx[..., 1::2]).contiguous()


def unpack_4bit(packed: Tensor, *, d: int) -> Tensor:
    if packed.size(-1) * 2 != d:
        raise ValueError(f"packed last dim {packed.size(-1)} * 2 != d={d}")
    return torch.stack([(packed >> 4) & 0xF, packed & 0xF], dim=-1).reshape(
        *packed.shape[:-1], d).contiguous()


def pack_2bit(idx: Tensor) -> Tensor:
    """(..., D) codes in [0, 4) -> (..., D/4) bytes, dim 4j at bits 7:6."""
    idx = idx.to(torch.uint8)
    if idx.size(-1) % 4:
        raise ValueError(f"2-bit pack requires last dim divisible by 4, got {idx.size(-1)}")
    return ((idx[..., 0::4] << 6) | (idx[..., 1::4] << 4) | (idx[..., 2::4] << 2)
            | idx[..., 3::4]).contiguous()


def unpack_2bit(packed: Tensor, *, d: int) -> Tensor:
    if packed.size(-1) * 4 != d:
        raise ValueError(f"packed last dim {packed.size(-1)} * 4 != d={d}")
    parts = [(packed >> s) & 0x3 for s in (6, 4, 2, 0)]
    return torch.stack(parts, dim=-1).reshape(*packed.shape[:-1], d).contiguous()


@dataclass(frozen=True)
class CompressedSlot:
    """Encoded rows: ``idx`` (..., D*bits/8) uint8 packed codes, ``norm`` (...,) fp32."""
    idx: Tensor
    norm: Tensor


class Compressor:
    """Rotation + codebook of one role (K or V); GPU encode/decode.

    Constructor arguments follow the reference (``compression.py:208-279``).
    """

    def __init__(self, dim: int, *, num_levels: int = 16, codebook: Optional[Tensor] = None,
                 rotation: Optional[Tensor] = None, codebook_mode: str = "lloyd_beta",
                 device: torch.device | str = "cpu"):
        if num_levels not in (4, 16):
            raise ValueError(f"num_levels must be 4 or 16 (got {num_levels})")
        self.dim = dim
        self.num_levels = num_levels
        self.bits = 4 if num_levels == 16 else 2
        self.dims_per_byte = 8 // self.bits
        self.bytes_per_row = dim // self.dims_per_byte
        self.codebook_mode = codebook_mode
        rotation = hadamard_matrix(dim, device=device) if rotation is None else rotation.to(device)
        if codebook is None:
            if codebook_mode == "uniform":
                codebook = uniform_centroids(num_levels, device=device)
            elif codebook_mode == "lloyd_beta":
                codebook = lloyd_max_centroids_beta(num_levels, dim, device=device)
            else:
                raise ValueError(f"unknown codebook_mode: {codebook_mode}")
        else:
            codebook = codebook.to(device)
        self.rotation = rotation.contiguous()
        self.codebook = codebook.contiguous()

    @property
    def device(self) -> torch.device:
        return self.rotation.device

    def to(self, device: torch.device | str) -> "Compressor":
        return Compressor(self.dim, num_levels=self.num_levels, codebook=self.codebook,
                          rotation=self.rotation, codebook_mode=self.codebook_mode,
                          device=device)

    def compression_ratio(self) -> float:
        return (self.dim * 2) / (self.dim * self.bits / 8 + 4)

    def encode(self, x: Tensor) -> CompressedSlot:
        """GPU encode of (..., D) fp16 rows with the fused HIP encoder.

        Uses the butterfly Hadamard of the paged encoder, so ``rotation`` must
        be the default Sylvester matrix.
        """
        from sub0_amd import _native
        if x.size(-1) != self.dim or self.dim != 128:
            raise ValueError(f"x last dim {x.size(-1)} != dim={self.dim} (128 supported)")
        if x.device.type != "cuda":
            raise ValueError("Compressor.encode runs on the GPU (no CPU path)")
        lead = x.shape[:-1]
        rows = x.reshape(-1, 1, self.dim).to(torch.float16).contiguous()
        n = rows.shape[0]
        kb = self.bytes_per_row
        slot_bytes = (2 * kb + 8 + 15) // 16 * 16
        cache = torch.zeros(n, 1, slot_bytes, dtype=torch.uint8, device=x.device)
        slots = torch.arange(n, dtype=torch.int32, device=x.device)
        cb = self.codebook.float().to(x.device)
        _native.paged_encode(rows, rows, slots, cache, cb, cb)
        idx = cache[:, 0, :kb].reshape(*lead, kb).contiguous()
        norm = cache[:, 0, 2 * kb:2 * kb + 4].contiguous().view(torch.float32).reshape(lead)
        return CompressedSlot(idx=idx, norm=norm.contiguous())

    def decode(self, slot: CompressedSlot, *, dtype: torch.dtype = torch.float16,
               rotated: bool = False) -> Tensor:
        """fp16(codebook[idx] * norm), optionally un-rotated (table lookup on device)."""
        if slot.idx.device.type != "cuda":
            raise ValueError("Compressor.decode runs on the GPU (no CPU path)")
        idx = (unpack_4bit if self.bits == 4 else unpack_2bit)(slot.idx, d=self.dim)
        cb = self.codebook.to(slot.idx.device)
        x_rot = (cb[idx.long()] * slot.norm.unsqueeze(-1)).to(torch.float16)
        if rotated:
            return x_rot.to(dtype)
        rot = self.rotation.to(slot.idx.device)
        return torch.matmul(x_rot.float(), rot.t()).to(dtype)
