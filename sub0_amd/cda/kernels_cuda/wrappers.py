"""Decode and encode entry points (drop-in for ``cda/kernels_cuda/wrappers.py``).

* :func:`decode_hmma_v1` -- split-K decode over the paged K4V4 cache,
  unrotated fp16 Q in, unrotated fp16 O written in place
  (reference ``wrappers.py:79-124``).
* :func:`paged_encode_fused_cuda` -- fused Hadamard + norm + quantise +
  scatter into the paged cache (reference ``wrappers.py:127-156``); accepts
  16-level (K4V4) and 4-level (K2V2) codebooks.
* :func:`hybrid_attn_v1` -- chunked prefill over a compressed prefix plus the
  chunk's fresh fp16 K/V with a log-sum-exp merge, the function the
  reference's raw-K/V prefill routes import
  (``vllm_integration/cda_attn_v2.py:1023-1060, 1474-1532``; its own wrapper
  was removed, ``wrappers.py:14-20``).

Argument checks and error types follow the reference.  The split size
(``_choose_tile_n``) is MI355X's own policy: it targets one 512-thread
workgroup per CU (256 CUs) instead of the reference's 2-blocks-per-SM rule, and it is what the kernel plans with when called
through these wrappers.
"""
from __future__ import annotations

import functools
import math
from typing import Optional

import torch
from torch import Tensor

from sub0_amd import _native
from sub0_amd.cda import _torch_ops  # noqa: F401  -- registers torch.ops.cda_hip
from sub0_amd.cda.kernels_cuda.hmma_loader import (
    load_decode_hmma,
    load_paged_encode_fused,
)


@functools.lru_cache(maxsize=8)
def _get_num_sms(device_idx: int) -> int:
    """Compute-unit count of the device (reference ``wrappers.py:35-38``)."""
    return torch.cuda.get_device_properties(device_idx).multi_processor_count


def _choose_tile_n(past_len: int, *, B: int = 1, H_q: int = 32, device_idx: int = 0,
                   group_size: int = 4) -> int:
    """Context tokens per split-K partition (reference ``wrappers.py:41-76``).

    MI355X policy (``cda_decode_plan`` in the HIP library): one workgroup
    covers 8 KV heads of one sequence; aim for one workgroup per CU, at least
    64 and at most 16384 tokens and at most 512 partitions per sequence,
    rounded to 32 tokens.
    ``device_idx`` is accepted for signature parity.
    """
    H_kv = max(1, H_q // group_size)
    tile, _ = _native.decode_plan(B, H_q, H_kv, int(past_len), 0)
    return tile


def decode_hmma_v1(
    Q_fp16: Tensor,           # (B, H_q, D) fp16 -- UNROTATED
    kv_cache: Tensor,         # (num_total_slots, H_kv, 144) uint8 K4V4
    block_table: Tensor,      # (B, max_blocks) int32
    seq_lens: Tensor,         # (B,) int32 -- full seq_len (past + 1)
    output: Tensor,           # (B, H_q, D) fp16 -- written in place
    *,
    cb_K: Tensor,
    cb_V: Tensor,
    rotation_fp32: Tensor,
    rotation_fp16: Tensor,
    group_size: int,
    block_size: int,
    scale: Optional[float] = None,
    max_seq_len: Optional[int] = None,
    qk_without_k_decode: bool = False,
) -> None:
    """Single-query split-K decode (K4V4), output written in place.

    Graph-capturable when ``max_seq_len`` is given (no host sync); the split-K
    workspace comes from the caching allocator on the current stream.

    ``qk_without_k_decode`` (no counterpart in the reference's wrapper): the
    score-domain QK of ``attention.py:101-187`` for caches whose K codebook
    is the 16-level uniform one -- scores from the integer codes and the K
    norm, V decoded as usual.  Needs 8 KV heads and 144-byte slots; a cb_K
    other than uniform_centroids(16) gives NaN output.
    """
    B, H_q, D = Q_fp16.shape
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    if max_seq_len is None:
        max_seq_len = int(seq_lens.max().item())

    mod = load_decode_hmma(k4v2=False, group_size=group_size)
    tile_N = _choose_tile_n(max_seq_len, B=B, H_q=H_q,
                            device_idx=Q_fp16.device.index or 0, group_size=group_size)
    if Q_fp16.dtype != torch.float16:
        Q_fp16 = Q_fp16.to(torch.float16)
    if output.dtype != torch.float16:
        raise ValueError("decode_hmma_v1 requires fp16 output buffer")
    if qk_without_k_decode:
        torch.ops.cda_hip.decode_uniform_qk(
            Q_fp16.contiguous(), kv_cache.view(-1, *kv_cache.shape[-2:]),
            block_table.to(torch.int32) if block_table.dtype != torch.int32 else block_table,
            seq_lens.to(torch.int32) if seq_lens.dtype != torch.int32 else seq_lens,
            cb_K.float().contiguous(), cb_V.float().contiguous(),
            rotation_fp32.float().contiguous(), output, group_size, block_size, tile_N,
            max_seq_len, scale)
        return

    mod.cda_decode_full_hmma_v3(
        Q_fp16.contiguous(),
        kv_cache,
        block_table.to(torch.int32) if block_table.dtype != torch.int32 else block_table,
        seq_lens.to(torch.int32) if seq_lens.dtype != torch.int32 else seq_lens,
        cb_K.float().contiguous(), cb_V.float().contiguous(),
        rotation_fp32.float().contiguous(), rotation_fp16.contiguous(),
        output,
        group_size, block_size, tile_N, max_seq_len, scale,
    )


def paged_encode_fused_cuda(
    K: Tensor,                      # (T, H_kv, D=128) fp16, UN-rotated
    V: Tensor,
    slot_mapping: Tensor,           # (T,) int32
    flat_cache: Tensor,             # (num_slots, H_kv, slot_w) uint8
    *,
    cb_K: Tensor,                   # (16,) or (4,) fp32
    cb_V: Tensor,
) -> None:
    """Fused Hadamard-128 + L2-norm + nearest-centroid + pack + paged scatter.

    MSB-first packing, eps = 1e-12, negative slots skipped.  The kernel
    rotates with the Sylvester matrix / sqrt(128) itself (no rotation
    argument), as the reference's does; codes and norms are bit-identical to
    the reference's torch encode (compression.py:315-335).
    """
    if K.dtype != torch.float16 or V.dtype != torch.float16:
        raise TypeError("K, V must be fp16")
    if flat_cache.dtype != torch.uint8:
        raise TypeError("flat_cache must be uint8")
    if K.shape[-1] != 128:
        raise ValueError(f"D must be 128, got {K.shape[-1]}")
    mod = load_paged_encode_fused()
    sm_i32 = (slot_mapping
              if slot_mapping.dtype == torch.int32
              else slot_mapping.to(torch.int32))
    mod.cda_paged_encode_fused(
        K.contiguous(), V.contiguous(), sm_i32, flat_cache,
        cb_K.float().contiguous(), cb_V.float().contiguous(),
    )


def hybrid_attn_v1(
    q: Tensor,                      # (T, H_q, D) fp16, unrotated
    k: Tensor,                      # (T, H_kv, D) fp16, the chunk's fresh K, unrotated
    v: Tensor,                      # (T, H_kv, D) fp16
    output: Tensor,                 # (T, H_q, D) fp16, written in place
    kv_cache_flat: Tensor,          # (num_slots, H_kv, 144) uint8 K4V4
    block_table: Tensor,            # (B, max_blocks) int32
    *,
    cu_seqlens_q: Tensor,           # (B+1,) int32
    seq_lens: Tensor,               # (B,) int32, prefix + chunk
    cb_K: Tensor,
    cb_V: Tensor,
    rotation_fp32: Optional[Tensor] = None,
    rotation_fp16: Optional[Tensor] = None,
    scale: Optional[float] = None,
    group_size: int = 4,
    block_size: int = 16,
    max_seq_len: Optional[int] = None,
    max_query_len: Optional[int] = None,
) -> None:
    """Causal chunked prefill: the chunk's queries attend to the compressed
    prefix of their sequence (keys ``[0, seq_lens[b] - q_len)`` from the paged
    cache) and to the chunk's own raw K/V (causal), merged by log-sum-exp
    (``attention.py:239-272``).  The chunk's K/V are rotated into the cache's
    frame with the Hadamard kernel (``fa2_cda.py:256-287``); the rotation
    matrices are implied by the kernels (Sylvester / sqrt(128)) and accepted
    for signature compatibility.  ``max_seq_len`` / ``max_query_len`` bound
    the split plan; without them the bounds are read from the metadata (one
    device-to-host copy)."""
    if q.dim() != 3 or k.dim() != 3 or v.dim() != 3:
        raise ValueError("q must be (T, H_q, D) and k, v (T, H_kv, D)")
    if k.shape != v.shape or k.shape[0] != q.shape[0]:
        raise ValueError("k and v must be (T, H_kv, D) with the T of q")
    if output.shape != q.shape or output.dtype != torch.float16:
        raise ValueError("output must be fp16 and shaped like q")
    T, H_q, D = q.shape
    H_kv = k.shape[1]
    if H_q != H_kv * int(group_size):
        raise ValueError(f"H_q={H_q} != H_kv * group_size = {H_kv * int(group_size)}")
    if D != 128:
        raise ValueError(f"D must be 128, got {D}")
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    B = int(cu_seqlens_q.numel()) - 1
    if B <= 0 or T == 0:
        return
    q16 = (q if q.dtype == torch.float16 else q.to(torch.float16)).contiguous()
    k16 = (k if k.dtype == torch.float16 else k.to(torch.float16)).contiguous()
    v16 = (v if v.dtype == torch.float16 else v.to(torch.float16)).contiguous()
    cu = cu_seqlens_q if cu_seqlens_q.dtype == torch.int32 else cu_seqlens_q.to(torch.int32)
    sl = seq_lens if seq_lens.dtype == torch.int32 else seq_lens.to(torch.int32)
    bt = block_table if block_table.dtype == torch.int32 else block_table.to(torch.int32)
    if max_query_len is None:
        max_query_len = int((cu[1:] - cu[:-1]).max().item())
    if max_seq_len is None:
        max_seq_len = int(sl[:B].max().item())
    kv = kv_cache_flat.view(-1, *kv_cache_flat.shape[-2:]) if kv_cache_flat.dim() == 4 \
        else kv_cache_flat
    out = output if output.is_contiguous() else torch.empty_like(output)
    torch.ops.cda_hip.prefill_hybrid(q16, k16, v16, kv, bt, cu.contiguous(), sl.contiguous(),
                                     cb_K.float().contiguous(), cb_V.float().contiguous(), out,
                                     int(block_size), int(max_query_len), int(max_seq_len),
                                     float(scale))
    if out is not output:
        output.copy_(out)


__all__ = [
    "decode_hmma_v1",
    "hybrid_attn_v1",
    "paged_encode_fused_cuda",
]
