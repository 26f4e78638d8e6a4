"""Score-domain attention on MI355X (the GPU form of two functions of
``cda/algorithm/attention.py``).

* :func:`qk_scores_uniform_4bit_without_k_decode` (reference
  ``attention.py:101-152``): fp32 scores
  ``norm[k] * ((Q_rot . code[k]) / 8 - 15/16 * sum(Q_rot)) * scale`` straight
  from the packed 4-bit K codes of the 16-level uniform codebook, through
  ``cda_qk_scores_uniform4`` (``torch.ops.cda_hip.qk_scores_uniform4``).
* :func:`attention_compressed_rotated_reference_qk_without_k_decode`
  (``attention.py:155-187``): those scores, softmax, and V decoded to
  fp16(cb_V[code] * norm) by ``cda_dequantize_rows``.

The tensors follow the reference's ``CompressedSlot`` layout (contiguous
``idx`` (B, H_kv, M_k, 64) uint8, ``norm`` (B, H_kv, M_k) fp32); they must be
on the GPU.  The paged decode with the same score-domain QK is
``decode_hmma_v1(..., qk_without_k_decode=True)``.
"""
from __future__ import annotations

import math
from typing import Optional

import torch
from torch import Tensor

from sub0_amd import _native
from sub0_amd.cda import _torch_ops  # noqa: F401  -- registers torch.ops.cda_hip
from sub0_amd.cda.algorithm.compression import CompressedSlot


def qk_scores_uniform_4bit_without_k_decode(
    Q_rot: Tensor,                    # (B, H_q, M_q, D), rotated frame
    K_slot: CompressedSlot,           # idx (B, H_kv, M_k, D//2), norm (B, H_kv, M_k)
    *,
    group_size: int,
    scale: Optional[float] = None,
    causal: bool = False,
    q_offset: int = 0,
    key_start: int = 0,
    key_end: Optional[int] = None,
) -> Tensor:
    """(B, H_q, M_q, key_end - key_start) fp32 scores without decoding K
    (argument checks and errors as ``attention.py:127-143``)."""
    B, H_q, M_q, D = Q_rot.shape
    H_kv = K_slot.idx.shape[1]
    if H_q != H_kv * group_size:
        raise ValueError(f"H_q={H_q} != H_kv * group_size = {H_kv * group_size}")
    if K_slot.idx.size(-1) * 2 != D:
        raise ValueError(f"K packed dim {K_slot.idx.size(-1)} does not match D={D}")
    n_keys = K_slot.norm.size(-1)
    if K_slot.idx.size(-2) != n_keys:
        raise ValueError("K_slot idx/norm key dimensions do not match")
    if key_end is None:
        key_end = n_keys
    if not (0 <= key_start <= key_end <= n_keys):
        raise ValueError(f"invalid key window [{key_start}, {key_end}) for length {n_keys}")
    if D != 128:
        raise ValueError(f"the MI355X kernel takes D=128, got {D}")
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    q = (Q_rot if Q_rot.dtype == torch.float16 else Q_rot.to(torch.float16)).contiguous()
    out = torch.empty(B, H_q, M_q, key_end - key_start, dtype=torch.float32, device=q.device)
    torch.ops.cda_hip.qk_scores_uniform4(q, K_slot.idx.contiguous(),
                                         K_slot.norm.float().contiguous(), out, int(group_size),
                                         float(scale), bool(causal), int(q_offset),
                                         int(key_start), int(key_end))
    return out


def attention_compressed_rotated_reference_qk_without_k_decode(
    Q_rot: Tensor,
    K_slot: CompressedSlot,
    V_slot: CompressedSlot,
    *,
    cb_V: Tensor,
    group_size: int,
    scale: Optional[float] = None,
    causal: bool = False,
    q_offset: int = 0,
    key_start: int = 0,
    key_end: Optional[int] = None,
) -> Tensor:
    """Score-domain QK, softmax, decoded V (``attention.py:155-187``); fp16
    (B, H_q, M_q, 128) in the rotated frame.  The reference takes the V
    ``Compressor``; here its codebook ``cb_V``."""
    n_k = K_slot.norm.size(-1)
    if V_slot.norm.size(-1) != n_k:
        raise ValueError(f"K/V key lengths differ: {n_k} vs {V_slot.norm.size(-1)}")
    if key_end is None:
        key_end = n_k
    if not (0 <= key_start <= key_end <= n_k):
        raise ValueError(f"invalid key window [{key_start}, {key_end}) for length {n_k}")
    scores = qk_scores_uniform_4bit_without_k_decode(
        Q_rot, K_slot, group_size=group_size, scale=scale, causal=causal,
        q_offset=q_offset, key_start=key_start, key_end=key_end)
    B, H_q, M_q, D = Q_rot.shape
    H_kv = V_slot.idx.shape[1]
    v_idx = V_slot.idx[:, :, key_start:key_end].contiguous()
    v_norm = V_slot.norm[:, :, key_start:key_end].float().contiguous()
    nk = key_end - key_start
    v = _native.dequantize_rows(v_idx.reshape(B * H_kv * nk, 1, -1),
                                v_norm.reshape(B * H_kv * nk, 1), cb_V.float().contiguous())
    v = v.view(B, H_kv, nk, D)
    p = torch.softmax(scores, dim=-1).view(B, H_kv, group_size, M_q, nk)
    out = torch.einsum("bhgmk,bhkd->bhgmd", p, v.float())
    return out.reshape(B, H_q, M_q, D).to(torch.float16)


__all__ = [
    "attention_compressed_rotated_reference_qk_without_k_decode",
    "qk_scores_uniform_4bit_without_k_decode",
]
