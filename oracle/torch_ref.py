"""torch-CPU restatement of the reference's algorithm path -- TEST AND
BASELINE INFRASTRUCTURE ONLY.

The same torch operations, in the same order and dtypes, as the reference's
pure-torch oracle, so that on the CPU it gives the reference's bits:

* ``rotate`` / ``unrotate``      cda/algorithm/compression.py:287-296
* ``quantize_unit``              cda/algorithm/compression.py:298-313
* ``encode``                     cda/algorithm/compression.py:315-335
* ``decode_rows``                cda/algorithm/compression.py:337-361
* ``pack4`` / ``unpack4``        cda/algorithm/compression.py:163-188
* ``gqa_attention``              cda/algorithm/attention.py:60-93
* ``attention_compressed``       cda/algorithm/attention.py:306-346, 426-482
* ``causal_mask``                cda/algorithm/attention.py:46-57
* ``qk_scores_uniform4``         cda/algorithm/attention.py:101-152
* ``attention_qk_uniform4``      cda/algorithm/attention.py:155-187

``bench.py`` times it as the CPU baseline ("the reference's CPU algorithm
path"), and tests/ pin it against the reference-written golden fixtures.
The product (sub0_amd/) never imports this module.
"""
from __future__ import annotations

import math

import torch


def hadamard(dim: int = 128) -> torch.Tensor:
    """Sylvester H_dim / sqrt(dim) in fp32 (compression.py:43-57)."""
    i = torch.arange(dim)
    parity = torch.zeros(dim, dim, dtype=torch.int64)
    bits = i.unsqueeze(1) & i.unsqueeze(0)
    while bool(bits.any()):
        parity ^= bits & 1
        bits = bits >> 1
    sign = 1.0 - 2.0 * parity.to(torch.float32)
    return sign / math.sqrt(dim)


def rotate(x: torch.Tensor, H: torch.Tensor) -> torch.Tensor:
    """fp32 matmul, result cast back to the input dtype (compression.py:287-291)."""
    return torch.matmul(x.float(), H).to(x.dtype)


def unrotate(x: torch.Tensor, H: torch.Tensor) -> torch.Tensor:
    return torch.matmul(x.float(), H.t()).to(x.dtype)


def quantize_unit(u: torch.Tensor, cb: torch.Tensor) -> torch.Tensor:
    """bucketize + neighbour compare, ties to the lower index (:298-313)."""
    L = cb.numel()
    hi = torch.bucketize(u.contiguous(), cb).clamp_(0, L - 1)
    lo = (hi - 1).clamp_(min=0)
    take_hi = (cb[hi] - u).abs_() < (u - cb[lo]).abs_()
    return torch.where(take_hi, hi, lo).to(torch.uint8)


def pack4(idx: torch.Tensor) -> torch.Tensor:
    return ((idx[..., 0::2] << 4) | idx[..., 1::2]).contiguous()


def unpack4(packed: torch.Tensor) -> torch.Tensor:
    pair = torch.stack([(packed >> 4) & 0xF, packed & 0xF], dim=-1)
    return pair.reshape(*packed.shape[:-1], packed.shape[-1] * 2).contiguous()


def encode(x: torch.Tensor, cb: torch.Tensor, H: torch.Tensor):
    """(codes, norm) of fp16 rows (…, 128), 16-level codebook (:315-335)."""
    xr = rotate(x, H).float()
    n = xr.norm(dim=-1).clamp_min(1e-12)
    u = (xr / n.unsqueeze(-1)).clamp_(-1.0, 1.0)
    return pack4(quantize_unit(u, cb)), n.contiguous()


def decode_rows(codes: torch.Tensor, norm: torch.Tensor, cb: torch.Tensor) -> torch.Tensor:
    """Rotated-frame rows fp16(cb[idx] * norm) (:337-361, rotated=True)."""
    return (cb[unpack4(codes).long()] * norm.unsqueeze(-1)).to(torch.float16)


def gqa_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, group_size: int,
                  scale: float | None = None) -> torch.Tensor:
    """fp32 GQA softmax attention, fp16 out (attention.py:60-93, non-causal)."""
    B, H_q, M_q, D = q.shape
    H_kv = k.shape[1]
    s = 1.0 / math.sqrt(D) if scale is None else scale
    qg = q.float().view(B, H_kv, group_size, M_q, D)
    logits = torch.einsum("bhgmd,bhkd->bhgmk", qg, k.float()) * s
    p = torch.softmax(logits, dim=-1)
    o = torch.einsum("bhgmk,bhkd->bhgmd", p, v.float())
    return o.reshape(B, H_q, M_q, D).to(torch.float16)


def attention_compressed(q: torch.Tensor, k_codes, k_norm, v_codes, v_norm,
                         cb: torch.Tensor, H: torch.Tensor, group_size: int) -> torch.Tensor:
    """Rotate q (fp16), decode K/V rows in the rotated frame (fp16), attend,
    unrotate O (attention.py:306-346, 426-482)."""
    q_rot = rotate(q, H)
    k = decode_rows(k_codes, k_norm, cb)
    v = decode_rows(v_codes, v_norm, cb)
    o_rot = gqa_attention(q_rot, k, v, group_size)
    return unrotate(o_rot, H).to(torch.float16)


def causal_mask(m_q: int, m_k: int, q_offset: int = 0) -> torch.Tensor:
    """(M_q, M_k) bool, key k visible to query q iff k <= q + q_offset (:46-57)."""
    q = torch.arange(m_q).unsqueeze(1) + q_offset
    k = torch.arange(m_k).unsqueeze(0)
    return k <= q


def qk_scores_uniform4(q_rot: torch.Tensor, k_idx: torch.Tensor, k_norm: torch.Tensor,
                       group_size: int, scale: float | None = None, causal: bool = False,
                       q_offset: int = 0, key_start: int = 0, key_end: int | None = None):
    """Score-domain QK for the 16-level uniform codebook (:101-152):
    norm * ((Q @ code) / 8 - 15/16 * sum(Q)) * scale, codes never decoded.
    q_rot (B, H_q, M_q, 128); k_idx (B, H_kv, M_k, 64) uint8; k_norm (B, H_kv,
    M_k).  Returns (B, H_kv, g, M_q, key_end - key_start) fp32."""
    B, H_q, M_q, D = q_rot.shape
    H_kv = k_idx.shape[1]
    n_keys = k_norm.shape[-1]
    if key_end is None:
        key_end = n_keys
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    kid = k_idx[..., key_start:key_end, :]
    kn = k_norm[..., key_start:key_end].float()
    codes = unpack4(kid).float()
    qg = q_rot.float().view(B, H_kv, group_size, M_q, D)
    q_code = torch.einsum("bhgmd,bhkd->bhgmk", qg, codes)
    q_sum = qg.sum(dim=-1).unsqueeze(-1)
    scores = kn.unsqueeze(2).unsqueeze(3) * (q_code * 0.125 - q_sum * 0.9375)
    scores = scores * scale
    if causal:
        mask = causal_mask(M_q, key_end - key_start, q_offset - key_start)
        scores = scores.masked_fill(~mask, float("-inf"))
    return scores


def attention_qk_uniform4(q_rot, k_idx, k_norm, v_idx, v_norm, cb_v, group_size,
                          scale=None, causal=False, q_offset=0, key_start=0, key_end=None):
    """Score-domain QK, softmax, decoded V (:155-187); fp16 (B, H_q, M_q, 128)
    in the rotated frame."""
    if key_end is None:
        key_end = k_norm.shape[-1]
    scores = qk_scores_uniform4(q_rot, k_idx[..., key_start:key_end, :],
                                k_norm[..., key_start:key_end], group_size, scale, causal,
                                q_offset - key_start if causal else q_offset)
    v = decode_rows(v_idx[..., key_start:key_end, :], v_norm[..., key_start:key_end], cb_v)
    p = torch.softmax(scores, dim=-1)
    B, H_q, M_q, D = q_rot.shape
    out = torch.einsum("bhgmk,bhkd->bhgmd", p, v.float())
    return out.reshape(B, H_q, M_q, D).to(torch.float16)
