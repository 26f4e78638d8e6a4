"""Python entry points of the FA2-fork comparator namespace, on this build's
kernels (drop-in for ``cda/kernels_vllm_fa2_fork/interface.py``).

The reference wraps its vLLM FlashAttention-2 fork; here the same four
functions call ``torch.ops._cda_vllm_fa2_fork_C`` (registered by
:mod:`sub0_amd.cda._torch_ops`), whose ops run the MI355X varlen attention
kernel and the fp16(cb[code] * norm) row dequantisation.  Signatures,
argument meanings and the errors for unsupported features follow the
reference (``interface.py:138-470``):

* ``dequantize_compressed_kv`` -- rotated-frame fp16 K/V from codes + norms;
* ``flash_attn_varlen_func`` -- vLLM's FA varlen ABI on dense fp16 K/V;
* ``flash_attn_varlen_compressed_kv_func`` -- dequantise, then attend;
* ``flash_attn_varlen_compressed_kv_fused_func`` -- compressed K/V, flat
  varlen or paged pools.

Differences, all explicit: inference only (dropout 0), no sliding window,
soft-capping, ALiBi, split-KV, FP8 descales or sink tokens
(``NotImplementedError``, as the reference for most of them);
``return_softmax_lse=True`` returns ``(out, softmax_lse)`` as the reference,
softmax_lse (H_q, total_q) fp32 (log of the sum of exp(scale * q.k) over each
query's visible keys, +inf where there are none); ``gqa_decode_swap`` is
accepted and has no effect (the varlen kernel serves a GQA group from one K/V
tile already); ``flash_attn_varlen_func`` takes contiguous K/V only (no
``block_table``).
"""
from __future__ import annotations

from typing import Sequence

import torch

from sub0_amd.cda import _torch_ops  # noqa: F401  -- registers the namespace

_NS = "_cda_vllm_fa2_fork_C"


def _ops():
    return getattr(torch.ops, _NS)


def _window(window_size: Sequence[int] | None) -> tuple[int, int]:
    if window_size is None:
        return -1, -1
    if len(window_size) != 2:
        raise ValueError("window_size must contain exactly two values")
    return int(window_size[0]), int(window_size[1])


def _inference_args(dropout_p: float, softmax_scale, head_dim: int):
    if dropout_p != 0.0:
        raise NotImplementedError("inference only: dropout_p must be 0")
    return float(softmax_scale) if softmax_scale is not None else head_dim ** -0.5


def _flat_kv(idx: torch.Tensor, norm: torch.Tensor, name: str):
    """Compressed K or V as (total_k, H_kv, code bytes) + (total_k, H_kv):
    a 3-D pool as given, or the reference compressor's (B, H_kv, N, bytes)
    slot in batch-major token order."""
    if idx.dim() == 3:
        if norm.dim() != 2:
            raise ValueError(f"{name}_norm must be (total_k, H_kv) for 3D idx")
        return idx.contiguous(), norm.contiguous()
    if idx.dim() == 4:
        if norm.dim() != 3 or tuple(idx.shape[:3]) != tuple(norm.shape):
            raise ValueError(f"{name}_idx (B, H_kv, N, D/2) and {name}_norm (B, H_kv, N) "
                             "shapes disagree")
        B, H, N, nb = idx.shape
        return (idx.transpose(1, 2).reshape(B * N, H, nb).contiguous(),
                norm.transpose(1, 2).reshape(B * N, H).contiguous())
    raise ValueError(f"{name}_idx must be 3D or 4D, got {idx.dim()}D")


def _pair(k_idx, k_norm, v_idx, v_norm):
    ki, kn = _flat_kv(k_idx, k_norm, "k")
    vi, vn = _flat_kv(v_idx, v_norm, "v")
    if ki.shape != vi.shape or kn.shape != vn.shape:
        raise ValueError("K/V idx or norm shapes differ after flattening")
    return ki, kn, vi, vn


def dequantize_compressed_kv(k_idx: torch.Tensor, k_norm: torch.Tensor, v_idx: torch.Tensor,
                             v_norm: torch.Tensor, cb_k: torch.Tensor,
                             cb_v: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Rotated-frame fp16 K and V, (total_k, H_kv, 128) each."""
    ki, kn, vi, vn = _pair(k_idx, k_norm, v_idx, v_norm)
    return _ops().dequantize_compressed_kv(ki, kn, vi, vn, cb_k.contiguous(), cb_v.contiguous())


def flash_attn_varlen_func(
    q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, max_seqlen_q: int,
    cu_seqlens_q: torch.Tensor, max_seqlen_k: int, cu_seqlens_k: torch.Tensor | None = None,
    seqused_k: torch.Tensor | None = None, q_v: torch.Tensor | None = None,
    dropout_p: float = 0.0, softmax_scale: float | None = None, causal: bool = False,
    window_size: Sequence[int] | None = None, softcap: float = 0.0,
    alibi_slopes: torch.Tensor | None = None, deterministic: bool = False,
    return_attn_probs: bool = False, block_table: torch.Tensor | None = None,
    return_softmax_lse: bool = False, out: torch.Tensor | None = None,
    scheduler_metadata: torch.Tensor | None = None, q_descale: torch.Tensor | None = None,
    k_descale: torch.Tensor | None = None, v_descale: torch.Tensor | None = None,
    num_splits: int = 0, fa_version: int | None = 2, s_aux: torch.Tensor | None = None,
    cp_world_size: int = 1, cp_rank: int = 0, cp_tot_seqused_k: torch.Tensor | None = None,
) -> torch.Tensor:
    """vLLM's FA varlen call on dense fp16 K/V (rotated frame or not: plain
    attention), causal with bottom-right alignment when ``causal``."""
    if fa_version not in (None, 2):
        raise ValueError(f"only fa_version=2 is provided, got {fa_version}")
    if cu_seqlens_k is None and seqused_k is None:
        raise ValueError("cu_seqlens_k or seqused_k must be provided")
    if cu_seqlens_k is not None and seqused_k is not None:
        raise ValueError("cu_seqlens_k and seqused_k cannot both be provided")
    if block_table is not None and seqused_k is None:
        raise ValueError("seqused_k must be provided when block_table is provided")
    if block_table is not None:
        raise NotImplementedError("paged dense K/V (block_table) is not supported")
    if q_v is not None or scheduler_metadata is not None or s_aux is not None:
        raise NotImplementedError("q_v, scheduler_metadata and sink tokens are not supported")
    if cp_world_size != 1 or cp_rank != 0 or cp_tot_seqused_k is not None:
        raise NotImplementedError("context-parallel arguments are not supported")
    if return_attn_probs:
        raise NotImplementedError("attention probabilities are not returned")
    fp8 = {getattr(torch, "float8_e4m3fn", None), getattr(torch, "float8_e5m2", None)}
    if any(d is not None and t.dtype in fp8 for t, d in ((q, q_descale), (k, k_descale),
                                                          (v, v_descale))):
        raise NotImplementedError("FP8 inputs are not supported")
    scale = _inference_args(dropout_p, softmax_scale, q.shape[-1])
    wl, wr = _window(window_size)
    if cu_seqlens_k is None:
        # The reference reaches K through block_table in this case.
        raise NotImplementedError("seqused_k without cu_seqlens_k addresses paged K/V, which "
                                  "is not supported")
    res = _ops().varlen_fwd(q, k, v, out, cu_seqlens_q, cu_seqlens_k, seqused_k, None, None,
                            alibi_slopes, int(max_seqlen_q), int(max_seqlen_k), 0.0, scale,
                            False, bool(causal), wl, wr, float(softcap), False, int(num_splits),
                            None)
    return (res[0], res[1]) if return_softmax_lse else res[0]


def flash_attn_varlen_compressed_kv_func(
    q: torch.Tensor, k_idx: torch.Tensor, k_norm: torch.Tensor, v_idx: torch.Tensor,
    v_norm: torch.Tensor, cb_k: torch.Tensor, cb_v: torch.Tensor, max_seqlen_q: int,
    cu_seqlens_q: torch.Tensor, max_seqlen_k: int, cu_seqlens_k: torch.Tensor, *,
    out: torch.Tensor | None = None, dropout_p: float = 0.0,
    softmax_scale: float | None = None, causal: bool = False,
    window_size: Sequence[int] | None = None, softcap: float = 0.0,
    alibi_slopes: torch.Tensor | None = None, return_softmax_lse: bool = False,
    num_splits: int = 0,
) -> torch.Tensor:
    """Compressed K/V (rotated frame) dequantised to fp16 rows, then the
    varlen attention: the two-step bridge."""
    scale = _inference_args(dropout_p, softmax_scale, q.shape[-1])
    wl, wr = _window(window_size)
    ki, kn, vi, vn = _pair(k_idx, k_norm, v_idx, v_norm)
    res = _ops().varlen_fwd_compressed_kv(q, ki, kn, vi, vn, cb_k.contiguous(),
                                          cb_v.contiguous(), out, cu_seqlens_q, cu_seqlens_k,
                                          alibi_slopes, int(max_seqlen_q), int(max_seqlen_k),
                                          0.0, scale, False, bool(causal), wl, wr,
                                          float(softcap), False, int(num_splits), None)
    return (res[0], res[1]) if return_softmax_lse else res[0]


def flash_attn_varlen_compressed_kv_fused_func(
    q: torch.Tensor, k_idx: torch.Tensor, k_norm: torch.Tensor, v_idx: torch.Tensor,
    v_norm: torch.Tensor, cb_k: torch.Tensor, cb_v: torch.Tensor, max_seqlen_q: int,
    cu_seqlens_q: torch.Tensor, max_seqlen_k: int, cu_seqlens_k: torch.Tensor | None = None, *,
    seqused_k: torch.Tensor | None = None, block_table: torch.Tensor | None = None,
    out: torch.Tensor | None = None, dropout_p: float = 0.0,
    softmax_scale: float | None = None, causal: bool = False,
    window_size: Sequence[int] | None = None, softcap: float = 0.0,
    alibi_slopes: torch.Tensor | None = None, return_softmax_lse: bool = False,
    num_splits: int = 0, gqa_decode_swap: bool | None = None, uniform_codebook: bool = False,
) -> torch.Tensor:
    """Compressed K/V as flat varlen rows, or as paged pools (num_blocks,
    block_size, H_kv, D/2) + (num_blocks, block_size, H_kv) with
    ``block_table`` and ``seqused_k``."""
    del gqa_decode_swap
    scale = _inference_args(dropout_p, softmax_scale, q.shape[-1])
    wl, wr = _window(window_size)
    if block_table is not None:
        if seqused_k is None:
            raise ValueError("seqused_k must be provided with block_table")
        if k_idx.dim() != 4 or v_idx.dim() != 4 or k_norm.dim() != 3 or v_norm.dim() != 3:
            raise ValueError("paged idx must be (num_blocks, block_size, H_kv, D/2), norms "
                             "(num_blocks, block_size, H_kv)")
        if k_idx.shape != v_idx.shape or k_norm.shape != v_norm.shape or \
                tuple(k_norm.shape) != tuple(k_idx.shape[:3]):
            raise ValueError("K/V idx or norm shapes disagree")
        ki, kn, vi, vn = (t.contiguous() for t in (k_idx, k_norm, v_idx, v_norm))
    else:
        if cu_seqlens_k is None and seqused_k is None:
            raise ValueError("cu_seqlens_k or seqused_k must be provided")
        ki, kn, vi, vn = _pair(k_idx, k_norm, v_idx, v_norm)
    if cu_seqlens_k is None:
        cu_seqlens_k = torch.zeros(cu_seqlens_q.numel(), dtype=torch.int32, device=q.device)
    res = _ops().varlen_fwd_compressed_kv_fused(
        q, ki, kn, vi, vn, cb_k.contiguous(), cb_v.contiguous(), out, cu_seqlens_q,
        cu_seqlens_k, seqused_k, block_table, alibi_slopes, int(max_seqlen_q),
        int(max_seqlen_k), 0.0, scale, False, bool(causal), wl, wr, float(softcap), False,
        int(num_splits), bool(uniform_codebook), None)
    return (res[0], res[1]) if return_softmax_lse else res[0]


def register_vllm_backend(slot: str = "CUSTOM") -> None:
    """The reference names a vLLM backend module of the fork that it does not
    ship; neither does this build."""
    raise ImportError(f"no FA2-fork vLLM backend in this build (slot {slot!r}); the CDA "
                      "backend is sub0_amd.cda.vllm_plugin")


__all__ = [
    "dequantize_compressed_kv",
    "flash_attn_varlen_compressed_kv_fused_func",
    "flash_attn_varlen_compressed_kv_func",
    "flash_attn_varlen_func",
    "register_vllm_backend",
]
