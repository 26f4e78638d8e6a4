"""Class-(a) decode comparators on MI355X: dequantise, then attend.

The reference measures CDA decode against two "dequantise + FlashAttention"
routes selected by ``CDA_DECODE_BACKEND`` (``cda_attn_v2.py:138-154,
1062-1250``; Table 2 of ``results/table2_compute_path_iso``):

* R2 ``dequant_fa2``: gather the active slots and dequantise them to dense
  fp16 rotated K/V in a separate kernel, rotate q with a separate transform,
  run a plain flash attention over the dense K/V, rotate the output back
  (``cda_attn_v2.py:1062-1184``).
* R1 ``fused_dequant_fa2``: a flash attention that dequantises each K/V tile
  of the compressed cache in on-chip memory (``cda_attn_v2.py:1186-1250``).

Here R2 is ``paged_cache_to_dense_rotated`` (gather + dequant in one kernel),
the Hadamard helper on q, PyTorch's ``scaled_dot_product_attention`` (the
ROCm flash / memory-efficient kernels) with a key-length mask, and the
Hadamard helper on the output; R1 is the compressed-tile flash-attention
kernel of the prefill path with one query per sequence (it rotates q and the
output in its prologue and epilogue).  Both compute the same quantity as the
CDA decode: fp16 q_rot, softmax attention over fp16(centroid * norm) K/V,
fp16 O_rot, fp16 output.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F
from torch import Tensor

from sub0_amd import _native
from sub0_amd.cda.kernels_cuda.fa2_cda import _hadamard_or_matmul, paged_cache_to_dense_rotated


def dequant_fa2_decode(q: Tensor, kv_cache: Tensor, block_table: Tensor, seq_lens: Tensor,
                       out: Tensor, *, cb_K: Tensor, cb_V: Tensor, rotation_fp32: Tensor,
                       block_size: int, max_seq_len: int, scale: float) -> Tensor:
    """R2: q (B, H_q, 128) fp16 unrotated -> out (B, H_q, 128) fp16."""
    B, H_q, D = q.shape
    kv = kv_cache.view(-1, *kv_cache.shape[-2:]) if kv_cache.dim() == 4 else kv_cache
    H_kv = kv.shape[-2]
    N = int(max_seq_len)
    k_rot, v_rot = paged_cache_to_dense_rotated(kv, block_table, seq_lens, cb_K=cb_K, cb_V=cb_V,
                                                block_size=block_size, max_seq_len=N)
    q_rot = _hadamard_or_matmul(q.contiguous(), rotation_fp32)
    k = k_rot.view(B, N, H_kv, D).transpose(1, 2)
    v = v_rot.view(B, N, H_kv, D).transpose(1, 2)
    # An empty sequence keeps key 0 visible: its dense row is zero, so the
    # output is zero (as the CDA decode writes) rather than a 0/0.
    n_vis = seq_lens.to(torch.int64).clamp(min=1)
    mask = torch.arange(N, device=q.device)[None, :] < n_vis[:, None]
    o_rot = F.scaled_dot_product_attention(q_rot.unsqueeze(2), k, v,
                                           attn_mask=mask[:, None, None, :], scale=scale,
                                           enable_gqa=H_q != H_kv)
    _hadamard_or_matmul(o_rot.squeeze(2).contiguous(), rotation_fp32, out=out)
    return out


def fused_dequant_fa2_decode(q: Tensor, kv_cache: Tensor, block_table: Tensor,
                             seq_lens: Tensor, out: Tensor, *, cb_K: Tensor, cb_V: Tensor,
                             block_size: int, scale: float) -> Tensor:
    """R1: the compressed-tile flash attention with one query per sequence."""
    B = q.shape[0]
    kv = kv_cache.view(-1, *kv_cache.shape[-2:]) if kv_cache.dim() == 4 else kv_cache
    cu_q = torch.arange(B + 1, dtype=torch.int32, device=q.device)
    sl = seq_lens.to(torch.int32) if seq_lens.dtype != torch.int32 else seq_lens
    bt = block_table.to(torch.int32) if block_table.dtype != torch.int32 else block_table
    _native.prefill_paged(q.contiguous(), kv, bt, cu_q, sl.contiguous(), cb_K, cb_V, out,
                          block_size=int(block_size), max_query_len=1, scale=float(scale))
    return out
