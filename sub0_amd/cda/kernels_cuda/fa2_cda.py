"""CDA prefill (drop-in for ``cda/kernels_cuda/fa2_cda.py``).

Same public functions and argument handling as the reference
(``fa2_cda.py:36-230``).  One causal flash-attention kernel on MFMA, with the
Hadamard rotation of Q in front and the inverse rotation of O behind, reads
its K/V tiles from one of two sources:

* compressed: 64-key tiles of the paged cache dequantised straight into LDS
  (no dense K/V in HBM);
* dense: the rotated fp16 K/V materialised first (the reference's stage-0
  bridge, ``paged_cache_to_dense_rotated``), then read as plain rows.

The dense bridge dequantises every key once, the compressed source once per
64-query block, so long query chunks favour the bridge and short ones (chunked
prefill over a long past) the compressed tiles.  Measured on MI355X (eager,
32/8 heads): 8 sequences of 2K-7.6K new tokens 2.57 ms compressed / 2.25 ms
dense; 512-query chunks over 5K-8K keys 0.70 / 0.64; 2048-query chunks over
16K keys 2.89 / 2.52; 64-query chunks over 4K keys 0.21 / 0.36; 16 queries
over 16K keys 0.49 / 0.69; 64 sequences of 64-256 tokens 0.14 / 0.15.  The
default (``CDA_PREFILL_SOURCE=auto``) takes the bridge when max_query_len >=
256 and the dense K/V fit in 4 GiB; ``compressed`` / ``dense`` force a
source.  ``return_dense_kv=True`` always takes the bridge and returns the
dense K/V.  The unfused path of the reference calls vLLM's FlashAttention
around two Hadamard transforms; here it computes the same quantity (fp16
q_rot, fp16 O_rot, fp16 output) with the same kernel.
"""
from __future__ import annotations

import math
import os
from typing import Optional

import torch
from torch import Tensor

from sub0_amd import _native
from sub0_amd.cda import _torch_ops  # noqa: F401  -- registers torch.ops.cda_hip
from sub0_amd.cda.kernels_cuda.hmma_loader import (
    load_fa2_cda_hadamard,
    load_fa2_cda_loader,
    load_fa2_cda_varlen_fused,
)


def _hadamard_or_matmul(x: Tensor, rotation_fp32: Tensor, *,
                        out: Optional[Tensor] = None) -> Tensor:
    """x @ H/sqrt(D) rounded to fp16 (fa2_cda.py:36-61): the Hadamard kernel
    for contiguous fp16 D=128 device tensors, a matmul with ``rotation_fp32``
    otherwise."""
    D = x.shape[-1]
    if (D == 128 and x.is_cuda and x.dtype == torch.float16 and x.is_contiguous()
            and (out is None or (out.is_cuda and out.dtype == torch.float16
                                 and out.is_contiguous()))):
        y = torch.empty_like(x) if out is None else out
        load_fa2_cda_hadamard().hadamard128_fp16(x, y, 1.0 / math.sqrt(D))
        return y
    y = torch.matmul(x.float(), rotation_fp32).to(torch.float16)
    if out is not None:
        out.copy_(y)
        return out
    return y


def paged_cache_to_dense_rotated(kv_cache: Tensor, block_table: Tensor, seq_lens: Tensor, *,
                                 cb_K: Tensor, cb_V: Tensor, block_size: int, max_seq_len: int,
                                 k4v2: bool = False) -> tuple[Tensor, Tensor]:
    """Dense rotated K/V ``(B * max_seq_len, H_kv, 128)`` fp16, zero past
    ``seq_lens[b]`` (fa2_cda.py:64-95)."""
    bt = block_table.to(torch.int32) if block_table.dtype != torch.int32 else block_table
    sl = seq_lens.to(torch.int32) if seq_lens.dtype != torch.int32 else seq_lens
    mod = load_fa2_cda_loader(k4v2=k4v2)
    return mod.cda_fa2_paged_cache_to_dense_rotated(kv_cache, bt, sl, cb_K.contiguous(),
                                                    cb_V.contiguous(), int(block_size),
                                                    int(max_seq_len))


_DENSE_MIN_QUERY_LEN = 256
_DENSE_MAX_BYTES = 4 << 30


def prefill_source(B: int, H_kv: int, max_query_len: int, max_seq_len: int) -> str:
    """K/V source of the prefill kernel for this call: "dense" or
    "compressed" (policy in the module docstring; host integers only, so the
    choice never synchronises with the GPU)."""
    mode = os.environ.get("CDA_PREFILL_SOURCE", "auto")
    if mode in ("dense", "compressed"):
        return mode
    if mode != "auto":
        raise ValueError(f"CDA_PREFILL_SOURCE must be auto, dense or compressed, not {mode!r}")
    dense_bytes = 2 * B * max_seq_len * H_kv * 128 * 2
    if max_query_len >= _DENSE_MIN_QUERY_LEN and dense_bytes <= _DENSE_MAX_BYTES:
        return "dense"
    return "compressed"


def fa2_cda_prefill_varlen_v1(
    Q_fp16: Tensor,           # (T, H_q, D) fp16, unrotated
    kv_cache: Tensor,         # (num_slots, H_kv, slot_w) uint8 K4V4
    block_table: Tensor,      # (B, max_blocks) int32
    cu_seqlens_q: Tensor,     # (B+1,) int32
    seq_lens: Tensor,         # (B,) int32, full key lengths
    output: Tensor,           # (T, H_q, D) fp16, written in place
    *,
    cb_K: Tensor,
    cb_V: Tensor,
    rotation_fp32: Tensor,
    group_size: int,
    block_size: int,
    max_query_len: int,
    max_seq_len: int,
    scale: Optional[float] = None,
    causal: bool = True,
    k4v2: bool = False,
    return_dense_kv: bool = False,
    fuse_fa2_epilogue: bool = False,
) -> tuple[Tensor, Tensor] | None:
    """Causal varlen prefill from the compressed cache (fa2_cda.py:98-230).
    Queries are the last ``cu_seqlens_q[b+1] - cu_seqlens_q[b]`` positions of
    each sequence; key k is visible to query i iff k <= i + seq_lens[b] -
    (its query count)."""
    if Q_fp16.dim() != 3:
        raise ValueError("Q_fp16 must be (T, H_q, D)")
    if output.shape != Q_fp16.shape:
        raise ValueError("output shape must match Q_fp16")
    if output.dtype != torch.float16:
        raise ValueError("output must be fp16")
    Q_in = Q_fp16 if Q_fp16.dtype == torch.float16 else Q_fp16.to(torch.float16)
    T, H_q, D = Q_in.shape
    B = int(cu_seqlens_q.numel()) - 1
    if B <= 0:
        return None
    if H_q % group_size != 0:
        raise ValueError("H_q must be divisible by group_size")
    if not causal:
        raise NotImplementedError("the MI355X prefill kernels are causal-only")
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    cu_q = cu_seqlens_q.to(torch.int32) if cu_seqlens_q.dtype != torch.int32 else cu_seqlens_q
    sl = seq_lens.to(torch.int32) if seq_lens.dtype != torch.int32 else seq_lens
    bt = block_table.to(torch.int32) if block_table.dtype != torch.int32 else block_table
    kv = kv_cache.view(-1, *kv_cache.shape[-2:]) if kv_cache.dim() == 4 else kv_cache
    out = output if output.is_contiguous() else torch.empty_like(output)
    # K4V2 caches are read through the dense bridge (the compressed-tile
    # kernel reads K4V4 slots).
    dense = return_dense_kv or k4v2 or prefill_source(B, kv.shape[-2], int(max_query_len),
                                                      int(max_seq_len)) == "dense"
    if dense:
        k_rot, v_rot = paged_cache_to_dense_rotated(kv, bt, sl, cb_K=cb_K, cb_V=cb_V,
                                                    block_size=block_size,
                                                    max_seq_len=max_seq_len, k4v2=k4v2)
        cu_k = torch.arange(0, B + 1, dtype=torch.int32, device=Q_in.device) * int(max_seq_len)
        load_fa2_cda_varlen_fused().cda_fa2_varlen_fwd_hadamard(
            Q_in.contiguous(), k_rot, v_rot, out, cu_q.contiguous(), cu_k, sl.contiguous(),
            int(max_query_len), int(max_seq_len), float(scale))
    else:
        load_fa2_cda_varlen_fused()      # same artefact family as the reference's fused path
        _native.prefill_paged(Q_in.contiguous(), kv, bt, cu_q.contiguous(), sl.contiguous(),
                              cb_K, cb_V, out, block_size=int(block_size),
                              max_query_len=int(max_query_len), scale=float(scale),
                              max_seq_len=int(max_seq_len))
    if out is not output:
        output.copy_(out)
    if return_dense_kv:
        return k_rot, v_rot
    return None


def _check_raw(Q_fp16: Tensor, K_fp16: Tensor, V_fp16: Tensor, output: Tensor,
               group_size: int, causal: bool, fn: str) -> tuple[int, int, int, int]:
    """Shape checks of the raw-K/V prefill functions (fa2_cda.py:395-420)."""
    if Q_fp16.dim() != 3:
        raise ValueError("Q_fp16 must be (T, H_q, D)")
    if K_fp16.dim() != 3 or V_fp16.dim() != 3:
        raise ValueError("K_fp16 and V_fp16 must be (T, H_kv, D)")
    if K_fp16.shape != V_fp16.shape:
        raise ValueError("K_fp16 and V_fp16 shapes must match")
    if output.shape != Q_fp16.shape:
        raise ValueError("output shape must match Q_fp16")
    if output.dtype != torch.float16:
        raise ValueError("output must be fp16")
    if not causal:
        raise NotImplementedError(f"{fn} is causal-only")
    T, H_q, D = Q_fp16.shape
    if K_fp16.shape[0] != T:
        raise ValueError("raw K/V must have the same token count as Q")
    if K_fp16.shape[2] != D:
        raise ValueError("Q/K/V head dimensions must match")
    H_kv = K_fp16.shape[1]
    if H_q != H_kv * int(group_size):
        raise ValueError("H_q must equal H_kv * group_size")
    return T, H_q, H_kv, D


def _fp16c(x: Tensor) -> Tensor:
    return (x if x.dtype == torch.float16 else x.to(torch.float16)).contiguous()


def fa2_raw_prefill_varlen_v1(
    Q_fp16: Tensor,           # (T, H_q, D) fp16, unrotated
    K_fp16: Tensor,           # (T, H_kv, D) fp16, fresh uncompressed K
    V_fp16: Tensor,           # (T, H_kv, D) fp16, fresh uncompressed V
    cu_seqlens_q: Tensor,     # (B+1,) int32
    output: Tensor,           # (T, H_q, D) fp16, written in place
    *,
    group_size: int,
    max_query_len: int,
    scale: Optional[float] = None,
    causal: bool = True,
) -> None:
    """No-past causal prefill over the raw Q/K/V, no rotation
    (fa2_cda.py:373-460: the reference calls vLLM's FlashAttention varlen
    forward with cu_seqlens_k = cu_seqlens_q).  The Hadamard rotation is
    orthonormal, so this equals attention in the rotated frame."""
    T, H_q, H_kv, D = _check_raw(Q_fp16, K_fp16, V_fp16, output, group_size, causal,
                                 "fa2_raw_prefill_varlen_v1")
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    B = int(cu_seqlens_q.numel()) - 1
    if B <= 0 or T == 0:
        return
    cu = (cu_seqlens_q if cu_seqlens_q.dtype == torch.int32
          else cu_seqlens_q.to(torch.int32)).contiguous()
    used = (cu[1:] - cu[:-1]).contiguous()
    out = output if output.is_contiguous() else torch.empty_like(output)
    torch.ops.cda_hip.varlen_fwd(_fp16c(Q_fp16), _fp16c(K_fp16), _fp16c(V_fp16), out, cu, cu,
                                 used, int(max_query_len), float(scale), True)
    if out is not output:
        output.copy_(out)


def fa2_cda_prefill_rawkv_varlen_v1(
    Q_fp16: Tensor,           # (T, H_q, D) fp16, unrotated
    K_fp16: Tensor,           # (T, H_kv, D) fp16, fresh uncompressed K
    V_fp16: Tensor,           # (T, H_kv, D) fp16, fresh uncompressed V
    cu_seqlens_q: Tensor,     # (B+1,) int32
    seq_lens: Tensor,         # (B,) int32, key lengths (= query lengths: no past)
    output: Tensor,           # (T, H_q, D) fp16, written in place
    *,
    rotation_fp32: Tensor,
    group_size: int,
    max_query_len: int,
    max_seq_len: int,
    scale: Optional[float] = None,
    causal: bool = True,
) -> None:
    """No-past prefill through the fused FA2-CDA kernel fed from the raw K/V
    (fa2_cda.py:290-370): K and V rotated to fp16(x H / sqrt(128)) by the
    Hadamard kernel (fa2_cda.py:256-287), then the fused kernel with the Q
    Hadamard prologue and the inverse rotation of O.  The rotated rows stay
    in their packed varlen order (cu_seqlens_k = cu_seqlens_q) instead of the
    reference's B x max_seq_len padding; chunks with a compressed prefix
    belong to :func:`hybrid_attn_v1`."""
    T, H_q, H_kv, D = _check_raw(Q_fp16, K_fp16, V_fp16, output, group_size, causal,
                                 "fa2_cda_prefill_rawkv_varlen_v1")
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    B = int(cu_seqlens_q.numel()) - 1
    if B <= 0 or T == 0:
        return
    if int(max_query_len) > int(max_seq_len):
        raise ValueError("raw K/V request length exceeds max_seq_len")
    k_rot = _hadamard_or_matmul(_fp16c(K_fp16), rotation_fp32)
    v_rot = _hadamard_or_matmul(_fp16c(V_fp16), rotation_fp32)
    cu = (cu_seqlens_q if cu_seqlens_q.dtype == torch.int32
          else cu_seqlens_q.to(torch.int32)).contiguous()
    sl = (seq_lens if seq_lens.dtype == torch.int32 else seq_lens.to(torch.int32)).contiguous()
    out = output if output.is_contiguous() else torch.empty_like(output)
    load_fa2_cda_varlen_fused().cda_fa2_varlen_fwd_hadamard(
        _fp16c(Q_fp16), k_rot, v_rot, out, cu, cu, sl, int(max_query_len), int(max_seq_len),
        float(scale))
    if out is not output:
        output.copy_(out)


__all__ = [
    "fa2_cda_prefill_rawkv_varlen_v1",
    "fa2_cda_prefill_varlen_v1",
    "fa2_raw_prefill_varlen_v1",
    "paged_cache_to_dense_rotated",
]
