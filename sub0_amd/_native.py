"""ctypes binding of libcda_hip.so (the C ABI declared in include/cda_hip.h).

torch is used only as device-memory and stream plumbing: tensors are passed
as raw pointers plus sizes, on ``torch.cuda.current_stream()``.  There is no
CPU fallback: if the library is missing, or a tensor is not on a GPU, the
call raises.
"""
from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch  # noqa: F401  -- must be loaded first so libamdhip64 resolves to torch's runtime

import os

# SUB0_AMD_LIB may name another build of the same library (A/B measurements).
LIB_PATH = Path(os.environ.get("SUB0_AMD_LIB") or
                Path(__file__).resolve().parent / "_lib" / "libcda_hip.so")

# Exported symbols (kept in sync with include/cda_hip.h; tests check both).
SYMBOLS = (
    "cda_hip_version",
    "cda_hip_last_error",
    "cda_decode_plan",
    "cda_decode_workspace_size",
    "cda_decode_full_hmma_v3",
    "cda_decode_set_timing_events",
    "cda_decode_set_stream_kernel",
    "cda_decode_set_fused_kernel",
    "cda_decode_fused_plan",
    "cda_decode_full_hmma_v3_k4v2",
    "cda_paged_encode_fused_k4v2",
    "cda_fa2_paged_cache_to_dense_rotated_k4v2",
    "cda_decode_noalloc_max_workspace",
    "cda_decode_full_hmma_v3_noalloc",
    "cda_paged_encode_fused",
    "cda_prefill_paged_hadamard",
    "cda_prefill_workspace_size",
    "cda_prefill_paged_hadamard_ws",
    "cda_fa2_varlen_fwd_hadamard",
    "cda_fa2_varlen_fwd",
    "cda_fa2_varlen_fwd_lse",
    "cda_dequantize_rows",
    "cda_fa2_paged_cache_to_dense_rotated",
    "cda_hadamard128_fp16",
    "cda_prefill_hybrid_workspace_size",
    "cda_prefill_hybrid_rawkv",
    "cda_decode_full_hmma_v3_uniform_qk",
    "cda_qk_scores_uniform4",
)


class NativeMissing(ImportError):
    """libcda_hip.so is not built (run ``python -m sub0_amd.build``)."""


class CdaError(RuntimeError):
    """A C-ABI entry point returned an error code."""


_lock = threading.Lock()
_lib = None

_P = ctypes.c_void_p
_I32 = ctypes.c_int
_I64 = ctypes.c_int64
_F32 = ctypes.c_float
_SZ = ctypes.c_size_t


def lib():
    """Load (once) and return the ctypes handle of libcda_hip.so."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.is_file():
            raise NativeMissing(
                f"{LIB_PATH} not found; build it with `python -m sub0_amd.build` "
                "(hipcc --offload-arch=gfx950)")
        L = ctypes.CDLL(str(LIB_PATH))
        L.cda_hip_version.restype = _I32
        L.cda_hip_version.argtypes = []
        L.cda_hip_last_error.restype = ctypes.c_char_p
        L.cda_hip_last_error.argtypes = []
        L.cda_decode_plan.restype = _I32
        L.cda_decode_plan.argtypes = [_I32, _I32, _I32, _I32, _I32,
                                      ctypes.POINTER(_I32), ctypes.POINTER(_I32)]
        L.cda_decode_workspace_size.restype = _SZ
        L.cda_decode_workspace_size.argtypes = [_I32, _I32, _I32, _I32, _I32]
        L.cda_decode_full_hmma_v3.restype = _I32
        L.cda_decode_full_hmma_v3.argtypes = [
            _P, _P, _I64, _I32, _I32, _P, _I32, _P, _P, _P, _I32, _P, _P, _P,
            _I32, _I32, _I32, _I32, _I32, _I32, _F32, _P, _SZ, _P]
        L.cda_decode_noalloc_max_workspace.restype = _SZ
        L.cda_decode_noalloc_max_workspace.argtypes = []
        L.cda_decode_full_hmma_v3_noalloc.restype = _I32
        L.cda_decode_full_hmma_v3_noalloc.argtypes = [
            _P, _P, _I64, _I32, _I32, _P, _I32, _P, _P, _P, _I32, _P, _P, _P,
            _I32, _I32, _I32, _I32, _I32, _I32, _F32, _P]
        L.cda_decode_set_timing_events.restype = _I32
        L.cda_decode_set_timing_events.argtypes = [_P, _P]
        L.cda_decode_set_stream_kernel.restype = _I32
        L.cda_decode_set_stream_kernel.argtypes = [_I32]
        L.cda_decode_set_fused_kernel.restype = _I32
        L.cda_decode_set_fused_kernel.argtypes = [_I32]
        L.cda_decode_fused_plan.restype = _I32
        L.cda_decode_fused_plan.argtypes = [_I32, _I32, _I32, ctypes.POINTER(_I32),
                                            ctypes.POINTER(_I32)]
        L.cda_decode_full_hmma_v3_k4v2.restype = _I32
        L.cda_decode_full_hmma_v3_k4v2.argtypes = [
            _P, _P, _I64, _I32, _I32, _P, _I32, _P, _P, _P, _P, _P, _P,
            _I32, _I32, _I32, _I32, _I32, _I32, _F32, _P, _SZ, _P]
        L.cda_paged_encode_fused_k4v2.restype = _I32
        L.cda_paged_encode_fused_k4v2.argtypes = [
            _P, _P, _I64, _I64, _P, _I64, _P, _I64, _I32, _I32, _P, _P, _P]
        L.cda_fa2_paged_cache_to_dense_rotated_k4v2.restype = _I32
        L.cda_fa2_paged_cache_to_dense_rotated_k4v2.argtypes = [
            _P, _I64, _I32, _I32, _P, _I32, _P, _I32, _P, _P, _I32, _I32, _P, _P, _P]
        L.cda_paged_encode_fused.restype = _I32
        L.cda_paged_encode_fused.argtypes = [
            _P, _P, _I64, _I64, _P, _I64, _P, _I64, _I32, _I32, _P, _P, _I32, _P]
        L.cda_prefill_paged_hadamard.restype = _I32
        L.cda_prefill_paged_hadamard.argtypes = [
            _P, _P, _I64, _I32, _I32, _P, _I32, _P, _P, _I32, _P, _P, _I32, _P, _I32, _I32,
            _I32, _I32, _F32, _P]
        L.cda_prefill_workspace_size.restype = _SZ
        L.cda_prefill_workspace_size.argtypes = [_I32, _I32, _I32, _I32, _I32, _I32]
        L.cda_prefill_paged_hadamard_ws.restype = _I32
        L.cda_prefill_paged_hadamard_ws.argtypes = [
            _P, _P, _I64, _I32, _I32, _P, _I32, _P, _P, _I32, _P, _P, _I32, _P, _I32, _I32,
            _I32, _I32, _I32, _F32, _P, _SZ, _P]
        L.cda_decode_full_hmma_v3_uniform_qk.restype = _I32
        L.cda_decode_full_hmma_v3_uniform_qk.argtypes = [
            _P, _P, _I64, _I32, _I32, _P, _I32, _P, _P, _P, _P, _P, _I32, _I32, _I32, _I32,
            _I32, _I32, _F32, _P, _SZ, _P]
        L.cda_qk_scores_uniform4.restype = _I32
        L.cda_qk_scores_uniform4.argtypes = [
            _P, _P, _P, _P, _I32, _I32, _I32, _I32, _I32, _I64, _I64, _I64, _I64, _F32, _I32,
            _P]
        L.cda_prefill_hybrid_workspace_size.restype = _SZ
        L.cda_prefill_hybrid_workspace_size.argtypes = [_I32, _I32, _I32, _I32, _I32, _I32]
        L.cda_prefill_hybrid_rawkv.restype = _I32
        L.cda_prefill_hybrid_rawkv.argtypes = [
            _P, _P, _P, _P, _I64, _I32, _I32, _P, _I32, _P, _P, _I32, _P, _P, _I32, _P, _I32,
            _I32, _I32, _I32, _I32, _F32, _P, _SZ, _P]
        L.cda_fa2_varlen_fwd_hadamard.restype = _I32
        L.cda_fa2_varlen_fwd_hadamard.argtypes = [
            _P, _P, _P, _P, _P, _P, _P, _I32, _I32, _I32, _I32, _I32, _I32, _F32, _P]
        L.cda_fa2_varlen_fwd.restype = _I32
        L.cda_fa2_varlen_fwd.argtypes = [
            _P, _P, _P, _P, _P, _P, _P, _I32, _I32, _I32, _I32, _I32, _F32, _I32, _P]
        L.cda_fa2_varlen_fwd_lse.restype = _I32
        L.cda_fa2_varlen_fwd_lse.argtypes = [
            _P, _P, _P, _P, _P, _P, _P, _I32, _I32, _I32, _I32, _I32, _F32, _I32, _P, _P]
        L.cda_dequantize_rows.restype = _I32
        L.cda_dequantize_rows.argtypes = [
            _P, _P, _I64, _I32, _P, _I32, _P, _I32, _P, _I32, _I32, _P, _P]
        L.cda_fa2_paged_cache_to_dense_rotated.restype = _I32
        L.cda_fa2_paged_cache_to_dense_rotated.argtypes = [
            _P, _I64, _I32, _I32, _P, _I32, _P, _I32, _P, _P, _I32, _I32, _I32, _P, _P, _P]
        L.cda_hadamard128_fp16.restype = _I32
        L.cda_hadamard128_fp16.argtypes = [_P, _P, _I64, _F32, _P]
        _lib = L
    return _lib


def _check(rc: int, what: str) -> None:
    if rc != 0:
        msg = lib().cda_hip_last_error().decode(errors="replace")
        if msg.startswith(what + ": "):
            msg = msg[len(what) + 2:]
        if rc == -1:
            raise ValueError(f"{what}: {msg}")
        raise CdaError(f"{what} failed ({rc}): {msg}")


def _ptr(t: torch.Tensor | None):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(device: torch.device):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _require_gpu(*ts: torch.Tensor) -> torch.device:
    dev = ts[0].device
    for t in ts:
        if t.device.type != "cuda":
            raise ValueError("CDA kernels run on the GPU only; got a tensor on " + str(t.device))
        if t.device != dev:
            raise ValueError(f"all tensors must be on one device ({t.device} vs {dev})")
    return dev


# ------------------------------------------------------------------ decode --

def decode_plan(B: int, H_q: int, H_kv: int, max_seq_len: int, tile_n: int = 0):
    tn, ns = _I32(0), _I32(0)
    _check(lib().cda_decode_plan(B, H_q, H_kv, max_seq_len, tile_n, ctypes.byref(tn),
                                 ctypes.byref(ns)), "cda_decode_plan")
    return tn.value, ns.value


def decode_fused_plan(B: int, H_kv: int, max_seq_len: int) -> tuple[int, int]:
    """(wave_tokens, n_splits) of the single-launch decode."""
    wt, ns = _I32(), _I32()
    _check(lib().cda_decode_fused_plan(B, H_kv, max_seq_len, ctypes.byref(wt), ctypes.byref(ns)),
           "cda_decode_fused_plan")
    return wt.value, ns.value


def decode_workspace_size(B: int, H_q: int, H_kv: int, max_seq_len: int, tile_n: int = 0) -> int:
    return int(lib().cda_decode_workspace_size(B, H_q, H_kv, max_seq_len, tile_n))


def decode(q: torch.Tensor, kv_cache: torch.Tensor, block_table: torch.Tensor,
           seq_lens: torch.Tensor, cb_k: torch.Tensor, cb_v: torch.Tensor,
           rot_f32: torch.Tensor, rot_f16: torch.Tensor | None, out: torch.Tensor, *,
           group_size: int, block_size: int, tile_n: int, max_seq_len: int, scale: float,
           workspace: torch.Tensor | None = None, uniform_qk: bool = False) -> None:
    """Split-K decode over the paged cache; ``out`` is written in place.

    q (B, H_q, 128) fp16; kv_cache (num_slots, H_kv, slot_bytes) uint8;
    block_table (B, W) int32; seq_lens (B,) int32; cb_* (16,) fp32;
    rot_f32 (128, 128) fp32; out (B, H_q, 128) fp16.

    ``uniform_qk``: score-domain QK (attention.py:101-152) for a cb_K equal to
    the 16-level uniform codebook, K4V4 144-byte slots and 8 KV heads; the
    kernel checks cb_K on the device and writes NaN if it differs.
    """
    dev = _require_gpu(q, kv_cache, block_table, seq_lens, cb_k, cb_v, rot_f32, out)
    if q.dtype != torch.float16 or out.dtype != torch.float16:
        raise TypeError("q and out must be fp16")
    if kv_cache.dtype != torch.uint8:
        raise TypeError("kv_cache must be uint8")
    if block_table.dtype != torch.int32 or seq_lens.dtype != torch.int32:
        raise TypeError("block_table and seq_lens must be int32")
    if cb_k.dtype != torch.float32 or cb_v.dtype != torch.float32 or rot_f32.dtype != torch.float32:
        raise TypeError("codebooks and rot_f32 must be fp32")
    if q.dim() != 3 or q.shape[-1] != 128 or not q.is_contiguous():
        raise ValueError("q must be a contiguous (B, H_q, 128) tensor")
    if out.shape != q.shape or not out.is_contiguous():
        raise ValueError("out must be a contiguous tensor shaped like q")
    if kv_cache.dim() != 3 or not kv_cache.is_contiguous():
        raise ValueError("kv_cache must be a contiguous (num_slots, H_kv, slot_bytes) tensor")
    if block_table.dim() != 2 or block_table.stride(1) != 1:
        raise ValueError("block_table must be (B, max_blocks) with unit inner stride")
    if rot_f32.shape != (128, 128) or not rot_f32.is_contiguous():
        raise ValueError("rot_f32 must be a contiguous (128, 128) tensor")
    k4v2 = (cb_k.numel(), cb_v.numel()) == (16, 4)
    if cb_k.numel() != cb_v.numel() and not k4v2:
        raise ValueError("cb_K and cb_V must have the same number of levels (or 16 and 4: the "
                         "K4V2 cache)")
    B, H_q, _ = q.shape
    num_slots, H_kv, slot_bytes = kv_cache.shape
    if block_table.shape[0] < B or seq_lens.numel() < B:
        raise ValueError("block_table / seq_lens have fewer rows than q")
    cb_k = cb_k.contiguous()
    cb_v = cb_k if cb_v.data_ptr() == cb_k.data_ptr() else cb_v.contiguous()
    need = decode_workspace_size(B, H_q, H_kv, max_seq_len, tile_n)
    if (workspace is None or workspace.device != dev
            or workspace.numel() - ((-workspace.data_ptr()) % 256) < need):
        workspace = torch.empty(need + 256, dtype=torch.uint8, device=dev)
    ws_ptr = workspace.data_ptr()
    pad = (-ws_ptr) % 256
    if uniform_qk:
        if cb_k.numel() != 16 or cb_v.numel() != 16:
            raise ValueError("the score-domain QK reads K4V4 caches (16-level codebooks)")
        rc = lib().cda_decode_full_hmma_v3_uniform_qk(
            _ptr(q), _ptr(kv_cache), num_slots, slot_bytes, H_kv, _ptr(block_table),
            block_table.stride(0), _ptr(seq_lens), _ptr(cb_k), _ptr(cb_v), _ptr(rot_f32),
            _ptr(out), B, H_q, int(group_size), int(block_size), int(tile_n), int(max_seq_len),
            float(scale), ctypes.c_void_p(ws_ptr + pad), workspace.numel() - pad, _stream(dev))
        _check(rc, "cda_decode_full_hmma_v3_uniform_qk")
        return
    if k4v2:
        rc = lib().cda_decode_full_hmma_v3_k4v2(
            _ptr(q), _ptr(kv_cache), num_slots, slot_bytes, H_kv, _ptr(block_table),
            block_table.stride(0), _ptr(seq_lens), _ptr(cb_k), _ptr(cb_v), _ptr(rot_f32),
            _ptr(rot_f16), _ptr(out), B, H_q, int(group_size), int(block_size), int(tile_n),
            int(max_seq_len), float(scale), ctypes.c_void_p(ws_ptr + pad),
            workspace.numel() - pad, _stream(dev))
        _check(rc, "cda_decode_full_hmma_v3_k4v2")
        return
    rc = lib().cda_decode_full_hmma_v3(
        _ptr(q), _ptr(kv_cache), num_slots, slot_bytes, H_kv, _ptr(block_table),
        block_table.stride(0), _ptr(seq_lens), _ptr(cb_k), _ptr(cb_v),
        cb_k.numel(), _ptr(rot_f32), _ptr(rot_f16), _ptr(out), B, H_q, int(group_size),
        int(block_size), int(tile_n), int(max_seq_len), float(scale),
        ctypes.c_void_p(ws_ptr + pad), workspace.numel() - pad, _stream(dev))
    _check(rc, "cda_decode_full_hmma_v3")


def qk_scores_uniform4(q_rot: torch.Tensor, k_idx: torch.Tensor, k_norm: torch.Tensor,
                       out: torch.Tensor, *, group_size: int, scale: float, causal: bool,
                       q_offset: int, key_start: int, key_end: int) -> None:
    """Score-domain QK over contiguous compressed K (``cda_qk_scores_uniform4``):
    q_rot (B, H_q, M_q, 128) fp16, k_idx (B, H_kv, M_k, 64) uint8, k_norm
    (B, H_kv, M_k) fp32 -> out (B, H_q, M_q, key_end - key_start) fp32."""
    dev = _require_gpu(q_rot, k_idx, k_norm, out)
    if q_rot.dtype != torch.float16 or k_idx.dtype != torch.uint8:
        raise TypeError("Q_rot must be fp16 and K idx uint8")
    if k_norm.dtype != torch.float32 or out.dtype != torch.float32:
        raise TypeError("K norm and the scores must be fp32")
    for t in (q_rot, k_idx, k_norm, out):
        if not t.is_contiguous():
            raise ValueError("Q_rot, K idx / norm and the scores must be contiguous")
    B, H_q, M_q, _ = q_rot.shape
    H_kv, M_k = k_idx.shape[1], k_idx.shape[2]
    if out.shape != (B, H_q, M_q, key_end - key_start):
        raise ValueError("scores must be (B, H_q, M_q, key_end - key_start)")
    rc = lib().cda_qk_scores_uniform4(
        _ptr(q_rot), _ptr(k_idx), _ptr(k_norm), _ptr(out), B, H_q, H_kv, M_q, int(group_size),
        M_k, int(key_start), int(key_end), int(q_offset), float(scale), int(bool(causal)),
        _stream(dev))
    _check(rc, "cda_qk_scores_uniform4")


def set_split_timing_events(start=None, stop=None) -> None:
    """Record two ``torch.cuda.Event`` around the split-K kernel of later
    decode calls on this thread (``None, None`` to stop)."""
    sp = None if start is None else ctypes.c_void_p(start.cuda_event)
    ep = None if stop is None else ctypes.c_void_p(stop.cuda_event)
    _check(lib().cda_decode_set_timing_events(sp, ep), "cda_decode_set_timing_events")


def set_stream_kernel(enable: bool) -> None:
    """Allow (default) or forbid the page-streaming decode kernel for later
    calls in this process; forbidding it always runs the general kernel."""
    _check(lib().cda_decode_set_stream_kernel(int(bool(enable))), "cda_decode_set_stream_kernel")


def set_fused_kernel(enable: bool) -> None:
    """Allow (default) or forbid the single-launch decode for later calls in
    this process; forbidding it keeps the rotate / split / combine launches."""
    _check(lib().cda_decode_set_fused_kernel(int(bool(enable))), "cda_decode_set_fused_kernel")


def decode_algorithmic_bytes(B: int, N: int, H_q: int = 32, H_kv: int = 8,
                             block_size: int = 16, slot_data: int = 136) -> int:
    """HBM bytes one decode step must move: codes + norms of every (token, KV
    head), Q in and O out (fp16), the block-table entries and seq_lens."""
    return (B * N * H_kv * slot_data + B * H_q * 128 * 2 * 2
            + B * ((N + block_size - 1) // block_size) * 4 + 4 * B)


# ------------------------------------------------------------------ encode --

def paged_encode(k: torch.Tensor, v: torch.Tensor, slot_mapping: torch.Tensor,
                 flat_cache: torch.Tensor, cb_k: torch.Tensor, cb_v: torch.Tensor) -> None:
    """Fused Hadamard + norm + quantise + pack + scatter into ``flat_cache``."""
    dev = _require_gpu(k, v, slot_mapping, flat_cache, cb_k, cb_v)
    if k.dtype != torch.float16 or v.dtype != torch.float16:
        raise TypeError("K, V must be fp16")
    if flat_cache.dtype != torch.uint8:
        raise TypeError("flat_cache must be uint8")
    if slot_mapping.dtype != torch.int32:
        raise TypeError("slot_mapping must be int32")
    if k.dim() != 3 or k.shape != v.shape:
        raise ValueError("K and V must be (T, H_kv, 128) tensors of one shape")
    if k.shape[-1] != 128:
        raise ValueError(f"D must be 128, got {k.shape[-1]}")
    if k.stride(2) != 1 or k.stride(1) != 128 or v.stride(2) != 1 or v.stride(1) != 128:
        raise ValueError("K and V need contiguous heads (stride (*, 128, 1))")
    if flat_cache.dim() != 3 or not flat_cache.is_contiguous():
        raise ValueError("flat_cache must be a contiguous (num_slots, H_kv, slot_bytes) tensor")
    T, H_kv, _ = k.shape
    if flat_cache.shape[1] != H_kv:
        raise ValueError("flat_cache head count does not match K")
    if slot_mapping.numel() < T:
        raise ValueError("slot_mapping shorter than the number of tokens")
    levels = cb_k.numel()
    if (levels, cb_v.numel()) == (16, 4):        # the legacy K4V2 slot
        rc = lib().cda_paged_encode_fused_k4v2(
            _ptr(k), _ptr(v), k.stride(0), v.stride(0), _ptr(slot_mapping.contiguous()), T,
            _ptr(flat_cache), flat_cache.shape[0], flat_cache.shape[2], H_kv,
            _ptr(cb_k.float().contiguous()), _ptr(cb_v.float().contiguous()), _stream(dev))
        _check(rc, "cda_paged_encode_fused_k4v2")
        return
    if cb_v.numel() != levels or levels not in (4, 16):
        raise ValueError("cb_K and cb_V must both have 16 (K4V4) or 4 (K2V2) levels, or 16 and "
                         "4 (K4V2)")
    rc = lib().cda_paged_encode_fused(
        _ptr(k), _ptr(v), k.stride(0), v.stride(0), _ptr(slot_mapping.contiguous()), T,
        _ptr(flat_cache), flat_cache.shape[0], flat_cache.shape[2], H_kv,
        _ptr(cb_k.float().contiguous()), _ptr(cb_v.float().contiguous()), levels, _stream(dev))
    _check(rc, "cda_paged_encode_fused")


# ----------------------------------------------------------------- prefill --

def _check_paged(kv_cache, block_table, seq_lens, cb_k, cb_v, allow_k4v2=False):
    if kv_cache.dtype != torch.uint8 or kv_cache.dim() != 3 or not kv_cache.is_contiguous():
        raise ValueError("kv_cache must be a contiguous uint8 (num_slots, H_kv, slot_bytes) tensor")
    if block_table.dtype != torch.int32 or block_table.dim() != 2 or block_table.stride(1) != 1:
        raise ValueError("block_table must be int32 (B, max_blocks) with unit inner stride")
    if seq_lens.dtype != torch.int32:
        raise TypeError("seq_lens must be int32")
    if allow_k4v2 and (cb_k.numel(), cb_v.numel()) == (16, 4):
        return
    if cb_k.numel() != 16 or cb_v.numel() != 16:
        raise ValueError("the prefill kernels read K4V4 caches (16-level codebooks)")


def prefill_paged(q: torch.Tensor, kv_cache: torch.Tensor, block_table: torch.Tensor,
                  cu_seqlens_q: torch.Tensor, seq_lens: torch.Tensor, cb_k: torch.Tensor,
                  cb_v: torch.Tensor, out: torch.Tensor, *, block_size: int,
                  max_query_len: int, scale: float, max_seq_len: int | None = None,
                  workspace: torch.Tensor | None = None) -> None:
    """Causal varlen prefill straight from the compressed paged cache with the
    Hadamard prologue/epilogue; ``out`` (T, H_q, 128) fp16 is written in place.

    With ``max_seq_len`` (an upper bound of ``seq_lens``) short query chunks
    over long contexts split their keys over more workgroups
    (``cda_prefill_paged_hadamard_ws``); ``workspace`` (uint8, reused when large
    enough) holds the partials, else one is allocated."""
    dev = _require_gpu(q, kv_cache, block_table, cu_seqlens_q, seq_lens, cb_k, cb_v, out)
    if q.dtype != torch.float16 or out.dtype != torch.float16:
        raise TypeError("Q and output must be fp16")
    if q.dim() != 3 or q.shape[-1] != 128 or not q.is_contiguous():
        raise ValueError("Q must be a contiguous (T, H_q, 128) tensor")
    if out.shape != q.shape or not out.is_contiguous():
        raise ValueError("output must be a contiguous tensor shaped like Q")
    if cu_seqlens_q.dtype != torch.int32:
        raise TypeError("cu_seqlens_q must be int32")
    _check_paged(kv_cache, block_table, seq_lens, cb_k, cb_v)
    T, H_q, _ = q.shape
    B = cu_seqlens_q.numel() - 1
    if seq_lens.numel() < B or block_table.shape[0] < B:
        raise ValueError("seq_lens / block_table have fewer rows than cu_seqlens_q")
    num_slots, H_kv, slot_bytes = kv_cache.shape
    need = 0
    if max_seq_len is not None:
        need = prefill_workspace_size(B, T, H_q, H_kv, int(max_query_len), int(max_seq_len))
    if need == 0:
        rc = lib().cda_prefill_paged_hadamard(
            _ptr(q), _ptr(kv_cache), num_slots, slot_bytes, H_kv, _ptr(block_table),
            block_table.stride(0), _ptr(cu_seqlens_q), _ptr(seq_lens), B,
            _ptr(cb_k.float().contiguous()), _ptr(cb_v.float().contiguous()), 16, _ptr(out), T,
            H_q, int(block_size), int(max_query_len), float(scale), _stream(dev))
        _check(rc, "cda_prefill_paged_hadamard")
        return
    if (workspace is None or workspace.device != dev
            or workspace.numel() - ((-workspace.data_ptr()) % 256) < need):
        workspace = torch.empty(need + 256, dtype=torch.uint8, device=dev)
    ws_ptr = workspace.data_ptr()
    pad = (-ws_ptr) % 256
    rc = lib().cda_prefill_paged_hadamard_ws(
        _ptr(q), _ptr(kv_cache), num_slots, slot_bytes, H_kv, _ptr(block_table),
        block_table.stride(0), _ptr(cu_seqlens_q), _ptr(seq_lens), B,
        _ptr(cb_k.float().contiguous()), _ptr(cb_v.float().contiguous()), 16, _ptr(out), T, H_q,
        int(block_size), int(max_query_len), int(max_seq_len), float(scale),
        ctypes.c_void_p(ws_ptr + pad), workspace.numel() - pad, _stream(dev))
    _check(rc, "cda_prefill_paged_hadamard_ws")


def prefill_workspace_size(B: int, T: int, H_q: int, H_kv: int, max_query_len: int,
                           max_seq_len: int) -> int:
    """Bytes of scratch the key-split prefill needs (0: it would not split)."""
    return int(lib().cda_prefill_workspace_size(B, T, H_q, H_kv, max_query_len, max_seq_len))


def prefill_hybrid(q: torch.Tensor, k_new: torch.Tensor, v_new: torch.Tensor,
                   kv_cache: torch.Tensor, block_table: torch.Tensor,
                   cu_seqlens_q: torch.Tensor, seq_lens: torch.Tensor, cb_k: torch.Tensor,
                   cb_v: torch.Tensor, out: torch.Tensor, *, block_size: int,
                   max_query_len: int, max_seq_len: int, scale: float,
                   workspace: torch.Tensor | None = None) -> None:
    """Chunked prefill over a compressed prefix plus the chunk's own fresh K/V
    (``cda_prefill_hybrid_rawkv``): the queries of sequence b are the last
    ``cu_seqlens_q[b+1] - cu_seqlens_q[b]`` of its ``seq_lens[b]`` positions;
    keys before the chunk come from the paged cache, the chunk's keys from
    ``k_new`` / ``v_new`` (T, H_kv, 128) fp16 (unrotated, causal), merged by
    log-sum-exp.  ``out`` (T, H_q, 128) fp16 is written in place."""
    dev = _require_gpu(q, k_new, v_new, kv_cache, block_table, cu_seqlens_q, seq_lens, cb_k,
                       cb_v, out)
    for t, nm in ((q, "Q"), (k_new, "K"), (v_new, "V"), (out, "output")):
        if t.dtype != torch.float16:
            raise TypeError(f"{nm} must be fp16")
        if t.dim() != 3 or t.shape[-1] != 128 or not t.is_contiguous():
            raise ValueError(f"{nm} must be a contiguous (T, heads, 128) tensor")
    if out.shape != q.shape:
        raise ValueError("output must be shaped like Q")
    if k_new.shape != v_new.shape or k_new.shape[0] != q.shape[0]:
        raise ValueError("K and V must be (T, H_kv, 128) with the T of Q")
    if cu_seqlens_q.dtype != torch.int32:
        raise TypeError("cu_seqlens_q must be int32")
    _check_paged(kv_cache, block_table, seq_lens, cb_k, cb_v)
    T, H_q, _ = q.shape
    B = cu_seqlens_q.numel() - 1
    if seq_lens.numel() < B or block_table.shape[0] < B:
        raise ValueError("seq_lens / block_table have fewer rows than cu_seqlens_q")
    num_slots, H_kv, slot_bytes = kv_cache.shape
    if k_new.shape[1] != H_kv:
        raise ValueError(f"K/V have {k_new.shape[1]} heads, the cache {H_kv}")
    if B == 0 or T == 0 or max_query_len <= 0:
        return
    need = int(lib().cda_prefill_hybrid_workspace_size(B, T, H_q, H_kv, int(max_query_len),
                                                        max(1, int(max_seq_len))))
    if need == 0:
        raise ValueError("unsupported hybrid prefill shape (H_q / H_kv must be 4 or 8)")
    if (workspace is None or workspace.device != dev
            or workspace.numel() - ((-workspace.data_ptr()) % 256) < need):
        workspace = torch.empty(need + 256, dtype=torch.uint8, device=dev)
    ws_ptr = workspace.data_ptr()
    pad = (-ws_ptr) % 256
    rc = lib().cda_prefill_hybrid_rawkv(
        _ptr(q), _ptr(k_new), _ptr(v_new), _ptr(kv_cache), num_slots, slot_bytes, H_kv,
        _ptr(block_table), block_table.stride(0), _ptr(cu_seqlens_q), _ptr(seq_lens), B,
        _ptr(cb_k.float().contiguous()), _ptr(cb_v.float().contiguous()), 16, _ptr(out), T, H_q,
        int(block_size), int(max_query_len), int(max_seq_len), float(scale),
        ctypes.c_void_p(ws_ptr + pad), workspace.numel() - pad, _stream(dev))
    _check(rc, "cda_prefill_hybrid_rawkv")


def fa2_varlen_fwd_hadamard(q: torch.Tensor, k_rot: torch.Tensor, v_rot: torch.Tensor,
                            out: torch.Tensor, cu_seqlens_q: torch.Tensor,
                            cu_seqlens_k: torch.Tensor, seqused_k: torch.Tensor,
                            max_query_len: int, max_seq_len: int, scale: float) -> None:
    """Causal varlen attention over dense rotated fp16 K/V rows with the
    Hadamard prologue on Q and the inverse rotation on O (the reference's
    cda_fa2_varlen_fwd_hadamard, fa2_cda.py:166-181)."""
    dev = _require_gpu(q, k_rot, v_rot, out, cu_seqlens_q, cu_seqlens_k, seqused_k)
    for t, nm in ((q, "Q"), (k_rot, "k_rot"), (v_rot, "v_rot"), (out, "output")):
        if t.dtype != torch.float16:
            raise TypeError(f"{nm} must be fp16")
        if t.dim() != 3 or t.shape[-1] != 128 or not t.is_contiguous():
            raise ValueError(f"{nm} must be a contiguous (rows, heads, 128) tensor")
    if k_rot.shape != v_rot.shape or out.shape != q.shape:
        raise ValueError("k_rot/v_rot and Q/output must have matching shapes")
    for t, nm in ((cu_seqlens_q, "cu_seqlens_q"), (cu_seqlens_k, "cu_seqlens_k"),
                  (seqused_k, "seqused_k")):
        if t.dtype != torch.int32:
            raise TypeError(f"{nm} must be int32")
    T, H_q, _ = q.shape
    B = cu_seqlens_q.numel() - 1
    rc = lib().cda_fa2_varlen_fwd_hadamard(
        _ptr(q), _ptr(k_rot), _ptr(v_rot), _ptr(out), _ptr(cu_seqlens_q),
        _ptr(cu_seqlens_k), _ptr(seqused_k), B, T, H_q, k_rot.shape[1], int(max_query_len),
        int(max_seq_len), float(scale), _stream(dev))
    _check(rc, "cda_fa2_varlen_fwd_hadamard")


def fa2_varlen_fwd(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, out: torch.Tensor,
                   cu_seqlens_q: torch.Tensor, cu_seqlens_k: torch.Tensor,
                   seqused_k: torch.Tensor, max_query_len: int, scale: float,
                   causal: bool, softmax_lse: torch.Tensor | None = None) -> None:
    """Varlen flash attention over dense fp16 K/V rows with no rotation: q, k,
    v and out all in one frame (the FA2 varlen forward the fork's
    comparator ops run).  Sequence b's keys are rows cu_seqlens_k[b] ..
    cu_seqlens_k[b] + seqused_k[b] - 1; causal = bottom-right aligned.
    With ``softmax_lse`` ((H_q, T) fp32) it also receives each query's
    log(sum exp(scale * q.k)) over its visible keys, +inf where none."""
    dev = _require_gpu(q, k, v, out, cu_seqlens_q, cu_seqlens_k, seqused_k)
    if softmax_lse is not None:
        _require_gpu(q, softmax_lse)
        if (softmax_lse.dtype != torch.float32 or not softmax_lse.is_contiguous()
                or tuple(softmax_lse.shape) != (q.shape[1], q.shape[0])):
            raise ValueError("softmax_lse must be a contiguous (H_q, T) fp32 tensor")
    for t, nm in ((q, "q"), (k, "k"), (v, "v"), (out, "out")):
        if t.dtype != torch.float16:
            raise TypeError(f"{nm} must be fp16")
        if t.dim() != 3 or t.shape[-1] != 128 or not t.is_contiguous():
            raise ValueError(f"{nm} must be a contiguous (rows, heads, 128) tensor")
    if k.shape != v.shape or out.shape != q.shape:
        raise ValueError("k/v and q/out must have matching shapes")
    for t, nm in ((cu_seqlens_q, "cu_seqlens_q"), (cu_seqlens_k, "cu_seqlens_k"),
                  (seqused_k, "seqused_k")):
        if t.dtype != torch.int32:
            raise TypeError(f"{nm} must be int32")
    T, H_q, _ = q.shape
    B = cu_seqlens_q.numel() - 1
    if softmax_lse is not None:
        rc = lib().cda_fa2_varlen_fwd_lse(
            _ptr(q), _ptr(k), _ptr(v), _ptr(out), _ptr(cu_seqlens_q), _ptr(cu_seqlens_k),
            _ptr(seqused_k), B, T, H_q, k.shape[1], int(max_query_len), float(scale),
            int(bool(causal)), _ptr(softmax_lse), _stream(dev))
        _check(rc, "cda_fa2_varlen_fwd_lse")
        return
    rc = lib().cda_fa2_varlen_fwd(
        _ptr(q), _ptr(k), _ptr(v), _ptr(out), _ptr(cu_seqlens_q), _ptr(cu_seqlens_k),
        _ptr(seqused_k), B, T, H_q, k.shape[1], int(max_query_len), float(scale),
        int(bool(causal)), _stream(dev))
    _check(rc, "cda_fa2_varlen_fwd")


def dequantize_rows(codes: torch.Tensor, norms: torch.Tensor, cb: torch.Tensor, *,
                    block_table: torch.Tensor | None = None,
                    seq_lens: torch.Tensor | None = None, block_size: int = 0,
                    max_seq_len: int = 0) -> torch.Tensor:
    """fp16(cb[code] * norm) rows (compression.py:337-361, rotated frame).

    codes (rows, H, 64 or 32) uint8, norms (rows, H) fp32 -> (rows, H, 128)
    fp16.  With a block table, codes/norms are a paged pool
    (num_blocks * block_size rows) and the result is (B * max_seq_len, H,
    128): sequence b's token t at row b * max_seq_len + t, zeros past
    seq_lens[b]."""
    dev = _require_gpu(codes, norms, cb)
    if codes.dtype != torch.uint8 or norms.dtype != torch.float32 or cb.dtype != torch.float32:
        raise TypeError("codes must be uint8, norms and cb fp32")
    codes = codes.contiguous()
    norms = norms.contiguous()
    H = codes.shape[-2]
    levels = cb.numel()
    if codes.shape[-1] != (64 if levels == 16 else 32):
        raise ValueError("codes must hold 64 (16 levels) or 32 (4 levels) bytes per row")
    if block_table is None:
        rows = codes.numel() // (H * codes.shape[-1])
        out = torch.empty(rows, H, 128, dtype=torch.float16, device=dev)
        rc = lib().cda_dequantize_rows(_ptr(codes), _ptr(norms), rows, H,
                                       _ptr(cb.contiguous()), levels, None, 0, None, 0, 0,
                                       _ptr(out), _stream(dev))
    else:
        if block_table.dtype != torch.int32 or seq_lens is None or seq_lens.dtype != torch.int32:
            raise TypeError("block_table and seq_lens must be int32")
        B = seq_lens.numel()
        rows = B * int(max_seq_len)
        out = torch.empty(rows, H, 128, dtype=torch.float16, device=dev)
        rc = lib().cda_dequantize_rows(_ptr(codes), _ptr(norms), rows, H,
                                       _ptr(cb.contiguous()), levels, _ptr(block_table),
                                       block_table.stride(0), _ptr(seq_lens), int(block_size),
                                       int(max_seq_len), _ptr(out), _stream(dev))
    _check(rc, "cda_dequantize_rows")
    return out


def paged_to_dense(kv_cache: torch.Tensor, block_table: torch.Tensor, seq_lens: torch.Tensor,
                   cb_k: torch.Tensor, cb_v: torch.Tensor, *, block_size: int,
                   max_seq_len: int) -> tuple[torch.Tensor, torch.Tensor]:
    """Dense rotated fp16 K/V, (B * max_seq_len, H_kv, 128) each, zero past
    seq_lens (fa2_cda.py:64-95)."""
    dev = _require_gpu(kv_cache, block_table, seq_lens, cb_k, cb_v)
    _check_paged(kv_cache, block_table, seq_lens, cb_k, cb_v, allow_k4v2=True)
    B = seq_lens.numel()
    num_slots, H_kv, slot_bytes = kv_cache.shape
    k_out = torch.empty(B * max_seq_len, H_kv, 128, dtype=torch.float16, device=dev)
    v_out = torch.empty_like(k_out)
    if (cb_k.numel(), cb_v.numel()) == (16, 4):  # the legacy K4V2 slot
        rc = lib().cda_fa2_paged_cache_to_dense_rotated_k4v2(
            _ptr(kv_cache), num_slots, slot_bytes, H_kv, _ptr(block_table),
            block_table.stride(0), _ptr(seq_lens), B, _ptr(cb_k.float().contiguous()),
            _ptr(cb_v.float().contiguous()), int(block_size), int(max_seq_len), _ptr(k_out),
            _ptr(v_out), _stream(dev))
        _check(rc, "cda_fa2_paged_cache_to_dense_rotated_k4v2")
        return k_out, v_out
    rc = lib().cda_fa2_paged_cache_to_dense_rotated(
        _ptr(kv_cache), num_slots, slot_bytes, H_kv, _ptr(block_table), block_table.stride(0),
        _ptr(seq_lens), B, _ptr(cb_k.float().contiguous()), _ptr(cb_v.float().contiguous()), 16,
        int(block_size), int(max_seq_len), _ptr(k_out), _ptr(v_out), _stream(dev))
    _check(rc, "cda_fa2_paged_cache_to_dense_rotated")
    return k_out, v_out


def hadamard128(x: torch.Tensor, y: torch.Tensor, scale: float) -> None:
    """y = fp16(scale * x @ H_128) row-wise (Sylvester order); x, y fp16 with a
    last dimension of 128."""
    dev = _require_gpu(x, y)
    if x.dtype != torch.float16 or y.dtype != torch.float16:
        raise TypeError("x and y must be fp16")
    if x.shape[-1] != 128 or x.shape != y.shape or not x.is_contiguous() or not y.is_contiguous():
        raise ValueError("x and y must be contiguous, of one shape, last dimension 128")
    rc = lib().cda_hadamard128_fp16(_ptr(x), _ptr(y), x.numel() // 128, float(scale), _stream(dev))
    _check(rc, "cda_hadamard128_fp16")
