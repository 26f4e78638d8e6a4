"""CDA attention backend for vLLM's v1 engine on MI355X
(drop-in for ``cda/kernels_cuda/vllm_integration/cda_attn_v2.py``).

The backend stores every token of every KV head in one 144-byte slot of the
paged cache and routes the three attention phases to the HIP kernels:

* cache update -> ``paged_encode_fused_cuda`` (Hadamard + L2 norm + 4-bit
  nearest centroid + scatter, one kernel);
* decode (one query per request) -> ``decode_hmma_v1`` (split-K over the
  compressed pages, rotation of Q and O fused in);
* prefill / chunked prefill -> ``fa2_cda_prefill_varlen_v1`` with the fused
  epilogue (causal flash attention over compressed tiles dequantised in LDS).

Slot layout (D = 128), ``cda_attn_v2.py:20-27, 52-60``::

    byte   0 ..  63   K codes, 4 bit, even dim in the high nibble
    byte  64 .. 127   V codes
    byte 128 .. 131   ||K|| fp32
    byte 132 .. 135   ||V|| fp32
    byte 136 .. 143   padding (rows stay 16-byte aligned)

vLLM allocates the cache as fp16 ``(num_blocks, block_size, H_kv, 72)``
(144 bytes per slot); :func:`_as_uint8_cache` reinterprets it as bytes.

vLLM is optional: the module imports and the backend classes are built with
plain stand-in base classes when vLLM is absent, so the dispatch can be
exercised with any object that carries the metadata fields.
"""
from __future__ import annotations

import atexit
import json
import os
import time
from dataclasses import dataclass
from typing import ClassVar

import torch

from sub0_amd.cda.algorithm.compression import Compressor

# ---------------------------------------------------------------------------
# Slot layout (cda_attn_v2.py:44-78)
# ---------------------------------------------------------------------------
HEAD_DIM = 128
_DATA_BYTES_PER_TOKEN = HEAD_DIM + 8                               # 136 payload bytes
_BYTES_PER_TOKEN = (_DATA_BYTES_PER_TOKEN + 15) // 16 * 16         # 144 allocated
_SLOT_FP16_ELEMS_COMPACT = _BYTES_PER_TOKEN // 2                   # 72 fp16 per slot
_SLOT_FP16_ELEMS_PER_TOKEN = 256                                   # vLLM's fp16 default


def _as_uint8_cache(kv_cache: torch.Tensor) -> torch.Tensor:
    """Byte view ``(num_blocks, block_size, H_kv, slot_bytes)`` of vLLM's
    fp16-typed cache: 72 fp16 -> 144 bytes, 256 fp16 -> 512 bytes
    (``cda_attn_v2.py:63-78``).  uint8 caches pass through."""
    if kv_cache.dtype == torch.uint8:
        return kv_cache
    num_blocks, block_size, num_kv_heads, last = kv_cache.shape
    if last == _SLOT_FP16_ELEMS_COMPACT:
        width = _BYTES_PER_TOKEN
    elif last == _SLOT_FP16_ELEMS_PER_TOKEN:
        width = 2 * _SLOT_FP16_ELEMS_PER_TOKEN
    else:
        raise ValueError(
            f"unexpected CDA cache last dim {last} "
            f"(expected {_SLOT_FP16_ELEMS_PER_TOKEN} or {_SLOT_FP16_ELEMS_COMPACT})")
    return kv_cache.view(torch.uint8).view(num_blocks, block_size, num_kv_heads, width)


# ---------------------------------------------------------------------------
# vLLM page-size accounting (cda_attn_v2.py:84-111)
# ---------------------------------------------------------------------------
def enable_cda_memory_saving() -> None:
    """Make vLLM size each page for 144-byte slots instead of fp16 K+V.

    Replaces ``real_page_size_bytes`` on vLLM's attention specs; idempotent.
    Needs vLLM (``ModuleNotFoundError`` otherwise)."""
    from vllm.v1.kv_cache_interface import (
        AttentionSpec,
        ChunkedLocalAttentionSpec,
        FullAttentionSpec,
        SlidingWindowSpec,
    )
    if getattr(AttentionSpec, "_cda_v2_patched", False):
        return

    def _page_bytes(self):
        return self.block_size * self.num_kv_heads * _BYTES_PER_TOKEN

    for cls in (AttentionSpec, FullAttentionSpec, ChunkedLocalAttentionSpec,
                SlidingWindowSpec):
        if "real_page_size_bytes" in cls.__dict__:
            cls.real_page_size_bytes = property(_page_bytes)
    AttentionSpec._cda_v2_patched = True


if os.environ.get("CDA_V2_ENABLE_MEMORY_SAVING") == "1":
    try:
        enable_cda_memory_saving()
    except ModuleNotFoundError:
        pass


# ---------------------------------------------------------------------------
# Per-call timing, CDA_V2_TIME_STEPS=1 (cda_attn_v2.py:112-297)
# ---------------------------------------------------------------------------
# Decode dispatch toggles are read once at import, as vLLM imports the backend
# before the engine starts (cda_attn_v2.py:126-154).
_USE_HMMA_V1 = os.environ.get("CDA_V2_USE_HMMA_V1") == "1"
_DECODE_BACKEND = os.environ.get("CDA_DECODE_BACKEND", "hmma_v1").lower()
_DUMP_EVERY = int(os.environ.get("CDA_V2_TIME_STEPS_DUMP_EVERY", "16"))
_TIMINGS: dict[str, list] = {}
_call_counter = [0]


def _time_steps_enabled() -> bool:
    return os.environ.get("CDA_V2_TIME_STEPS") == "1"


def _time_steps_out() -> str:
    prefix = os.environ.get("CDA_V2_TIME_STEPS_OUT", "/tmp/cda_v2_step_timings")
    return f"{prefix}.pid{os.getpid()}.json"


def _capturing() -> bool:
    return torch.cuda.is_available() and torch.cuda.is_current_stream_capturing()


def _summarise(values: list[float]) -> dict:
    warm = values[2:] if len(values) > 2 else values       # first calls: warm-up / capture
    if not warm:
        return {}
    s = sorted(warm)
    return {"mean": sum(warm) / len(warm), "min": s[0], "max": s[-1],
            "p50": s[len(s) // 2], "sum": sum(warm), "n": len(warm)}


def _dump_timings() -> None:
    """Write per-label CPU and device milliseconds to ``_time_steps_out()``."""
    if not _time_steps_enabled() or _capturing():
        return
    if any(e[1] is not None for rows in _TIMINGS.values() for e in rows):
        torch.cuda.synchronize()
    summary = {}
    for label, rows in _TIMINGS.items():
        if not rows:
            continue
        cpu = [r[0] for r in rows]
        dev = [r[1][0].elapsed_time(r[1][1]) for r in rows if r[1] is not None]
        summary[label] = {"n_total": len(rows), "cpu_ms": _summarise(cpu),
                          "device_ms": _summarise(dev)}
    path = _time_steps_out()
    if os.path.dirname(path):
        os.makedirs(os.path.dirname(path), exist_ok=True)
    with open(path, "w") as f:
        json.dump({"pid": os.getpid(), "call_count": _call_counter[0],
                   "summary": summary}, f, indent=2)


def _time_call(label: str, fn):
    """``fn()``; with CDA_V2_TIME_STEPS=1 also records its CPU time and,
    outside graph capture, its device time between two events."""
    if not _time_steps_enabled():
        return fn()
    events = None
    if torch.cuda.is_available() and not _capturing():
        events = (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
        events[0].record()
    t0 = time.perf_counter()
    try:
        return fn()
    finally:
        cpu_ms = (time.perf_counter() - t0) * 1e3
        if events is not None:
            events[1].record()
        _TIMINGS.setdefault(label, []).append((cpu_ms, events))
        _call_counter[0] += 1
        if _DUMP_EVERY > 0 and _call_counter[0] % _DUMP_EVERY == 0:
            _dump_timings()


atexit.register(_dump_timings)


# ---------------------------------------------------------------------------
# Codebooks and rotations, one set per device (cda_attn_v2.py:302-337)
# ---------------------------------------------------------------------------
_COMPRESSOR_CACHE: dict = {}
_HMMA_ARTIFACTS_CACHE: dict = {}


def _device_key(device: torch.device):
    device = torch.device(device)
    return device.type, device.index


def _get_compressors(device: torch.device) -> tuple[Compressor, Compressor]:
    """The K and V compressors (16-level Lloyd codebook, Hadamard rotation)
    of ``device``, built once."""
    key = _device_key(device)
    pair = _COMPRESSOR_CACHE.get(key)
    if pair is None:
        pair = (Compressor(HEAD_DIM, num_levels=16, device=device),
                Compressor(HEAD_DIM, num_levels=16, device=device))
        _COMPRESSOR_CACHE[key] = pair
    return pair


def _get_hmma_artifacts(cmp_K: Compressor, cmp_V: Compressor, device):
    """``(cb_K, cb_V, rotation_fp32, rotation_fp16)`` as the kernels take them,
    cached per compressor pair and device."""
    key = (id(cmp_K), id(cmp_V)) + _device_key(device)
    art = _HMMA_ARTIFACTS_CACHE.get(key)
    if art is None:
        r32 = cmp_K.rotation.float().contiguous()
        cb_K = cmp_K.codebook.float().contiguous()
        cb_V = cmp_V.codebook.float().contiguous()
        if cb_V.shape == cb_K.shape and torch.equal(cb_V, cb_K):
            cb_V = cb_K        # one table: lets the decode take its page-streaming kernel
        art = (cb_K, cb_V, r32, r32.to(torch.float16).contiguous())
        _HMMA_ARTIFACTS_CACHE[key] = art
    return art


# ---------------------------------------------------------------------------
# Metadata (cda_attn_v2.py:343-383)
# ---------------------------------------------------------------------------
@dataclass
class CDAv2AttentionMetadata:
    num_actual_tokens: int
    num_reqs: int
    max_query_len: int
    max_seq_len: int
    query_start_loc: torch.Tensor     # (num_reqs + 1,) int32
    seq_lens: torch.Tensor            # (num_reqs,) int32, keys incl. this step's tokens
    block_table: torch.Tensor         # (num_reqs, max_blocks) int32
    slot_mapping: torch.Tensor        # (num_actual_tokens,) int
    causal: bool = True
    dcp_world_size: int = 1
    dcp_rank: int = 0
    # Batches are ordered decode requests first, then prefill requests.
    num_prefill_tokens: int = 0
    num_decode_tokens: int = 0
    num_prefills: int = 0
    num_decodes: int = 0


def _split_counts_from_query_start(query_start_loc, num_reqs: int, num_actual_tokens: int,
                                   max_query_len: int) -> tuple[int, int, int, int]:
    """``(num_decodes, num_prefills, num_decode_tokens, num_prefill_tokens)``
    of a decode-first batch: the leading requests with at most one query token
    are decodes (``cda_attn_v2.py:366-383``)."""
    if max_query_len <= 1:
        return num_reqs, 0, num_actual_tokens, 0
    qs = query_start_loc.tolist() if isinstance(query_start_loc, torch.Tensor) \
        else list(query_start_loc)
    nd = 0
    while nd < num_reqs and int(qs[nd + 1]) - int(qs[nd]) <= 1:
        nd += 1
    nd_tok = int(qs[nd]) if nd else 0
    return nd, num_reqs - nd, nd_tok, num_actual_tokens - nd_tok


def _fp16_view(output: torch.Tensor, T: int, H_q: int, D: int):
    """A (T, H_q, D) view of ``output`` the kernels can write, or None."""
    if output.dtype != torch.float16 or not output.is_contiguous() or output.shape[0] < T:
        return None
    if output.dim() == 3 and output.shape[1] == H_q and output.shape[2] == D:
        return output[:T]
    if output.dim() == 2 and output.shape[1] == H_q * D:
        return output[:T].view(T, H_q, D)
    return None


def _copy_out(output: torch.Tensor, out: torch.Tensor, T: int) -> None:
    if output.dim() == 3:
        output[:T].copy_(out.to(output.dtype))
    else:
        output[:T].copy_(out.reshape(T, -1).to(output.dtype))


_PREFILL_FUSED = ("fa2_cda_fused", "fa2_cda_auto", "fa2_cda_direct", "fa2_cda_direct_v2")
_PREFILL_UNFUSED = ("fa2_cda",)
_PREFILL_RAWKV = ("fa2_rawkv", "fa2_cda_rawkv", "fa2_cda_fused_rawkv")


# ---------------------------------------------------------------------------
# Backend classes (cda_attn_v2.py:389-1705)
# ---------------------------------------------------------------------------
def _vllm_bases():
    """vLLM's backend base classes, or stand-ins with the same names."""
    try:
        from vllm.config import VllmConfig
        from vllm.v1.attention.backend import (
            AttentionBackend,
            AttentionCGSupport,
            AttentionImpl,
            AttentionMetadata,
            AttentionMetadataBuilder,
            AttentionType,
            CommonAttentionMetadata,
            MultipleOf,
        )
        from vllm.v1.kv_cache_interface import AttentionSpec
        return dict(AttentionBackend=AttentionBackend, AttentionCGSupport=AttentionCGSupport,
                    AttentionImpl=AttentionImpl, AttentionMetadata=AttentionMetadata,
                    AttentionMetadataBuilder=AttentionMetadataBuilder,
                    AttentionType=AttentionType,
                    CommonAttentionMetadata=CommonAttentionMetadata, MultipleOf=MultipleOf,
                    AttentionSpec=AttentionSpec, VllmConfig=VllmConfig, vllm=True)
    except ModuleNotFoundError:
        pass

    class _Generic:
        def __init__(self, *args, **kwargs):
            pass

        def __class_getitem__(cls, item):
            return cls

    class AttentionType:
        DECODER = "decoder"

    class AttentionCGSupport:
        UNIFORM_BATCH = "uniform_batch"

    class MultipleOf(int):
        pass

    return dict(AttentionBackend=type("AttentionBackend", (), {}),
                AttentionCGSupport=AttentionCGSupport,
                AttentionImpl=type("AttentionImpl", (_Generic,), {}),
                AttentionMetadata=type("AttentionMetadata", (), {}),
                AttentionMetadataBuilder=type("AttentionMetadataBuilder", (_Generic,), {}),
                AttentionType=AttentionType,
                CommonAttentionMetadata=type("CommonAttentionMetadata", (), {}),
                MultipleOf=MultipleOf, AttentionSpec=type("AttentionSpec", (), {}),
                VllmConfig=type("VllmConfig", (), {}), vllm=False)


_CLASSES = None


def _build_backend_classes():
    """``(Backend, Impl, MetadataBuilder, Metadata)`` on vLLM's base classes
    when vLLM is importable, on stand-ins otherwise.  Built once."""
    global _CLASSES
    if _CLASSES is not None:
        return _CLASSES
    b = _vllm_bases()
    AttentionType = b["AttentionType"]
    MultipleOf = b["MultipleOf"]
    have_vllm = b["vllm"]

    @dataclass
    class CDAv2AttentionMetadataVLLM(b["AttentionMetadata"]):
        num_actual_tokens: int
        num_reqs: int
        max_query_len: int
        max_seq_len: int
        query_start_loc: torch.Tensor
        seq_lens: torch.Tensor
        block_table: torch.Tensor
        slot_mapping: torch.Tensor
        causal: bool = True
        dcp_world_size: int = 1
        dcp_rank: int = 0
        num_prefill_tokens: int = 0
        num_decode_tokens: int = 0
        num_prefills: int = 0
        num_decodes: int = 0

    class CDAv2AttentionMetadataBuilder(
            b["AttentionMetadataBuilder"][CDAv2AttentionMetadataVLLM]):
        """Builds the metadata from vLLM's common metadata
        (``cda_attn_v2.py:475-550``).  Decode is graph-capturable
        (UNIFORM_BATCH); batches are reordered decode-first."""
        _cudagraph_support: ClassVar = b["AttentionCGSupport"].UNIFORM_BATCH
        reorder_batch_threshold: int | None = 1

        @classmethod
        def get_cudagraph_support(cls, vllm_config, kv_cache_spec):
            return cls._cudagraph_support

        def __init__(self, kv_cache_spec, layer_names, vllm_config, device) -> None:
            super().__init__(kv_cache_spec, layer_names, vllm_config, device)
            self.dcp_world_size, self.dcp_rank = 1, 0
            try:
                from vllm.distributed.parallel_state import get_dcp_group
                grp = get_dcp_group()
                self.dcp_world_size, self.dcp_rank = grp.world_size, grp.rank_in_group
            except (AssertionError, ImportError):
                pass

        def build(self, common_prefix_len: int, common_attn_metadata,
                  fast_build: bool = False) -> CDAv2AttentionMetadataVLLM:
            c = common_attn_metadata
            try:
                from vllm.v1.attention.backends.utils import split_decodes_and_prefills
                counts = split_decodes_and_prefills(c, decode_threshold=1)
            except Exception:
                counts = _split_counts_from_query_start(
                    getattr(c, "query_start_loc_cpu", c.query_start_loc),
                    c.num_reqs, c.num_actual_tokens, c.max_query_len)
            nd, npf, nd_tok, np_tok = counts
            return CDAv2AttentionMetadataVLLM(
                num_actual_tokens=c.num_actual_tokens, num_reqs=c.num_reqs,
                max_query_len=c.max_query_len, max_seq_len=c.max_seq_len,
                query_start_loc=c.query_start_loc, seq_lens=c.seq_lens,
                block_table=c.block_table_tensor, slot_mapping=c.slot_mapping,
                causal=getattr(c, "causal", True),
                dcp_world_size=self.dcp_world_size, dcp_rank=self.dcp_rank,
                num_prefill_tokens=np_tok, num_decode_tokens=nd_tok,
                num_prefills=npf, num_decodes=nd)

    class CDAv2AttentionBackend(b["AttentionBackend"]):
        """Backend descriptor (``cda_attn_v2.py:552-614``)."""
        accept_output_buffer: bool = True
        supported_dtypes: ClassVar[list] = [torch.float16]
        supported_kv_cache_dtypes: ClassVar[list] = ["auto", "uint8"]
        forward_includes_kv_cache_update: bool = False

        @staticmethod
        def get_supported_kernel_block_sizes() -> list:
            return [MultipleOf(16)]

        @staticmethod
        def get_name() -> str:
            return "CDA"

        @staticmethod
        def get_impl_cls() -> type:
            return CDAv2AttentionImpl

        @staticmethod
        def get_builder_cls() -> type:
            return CDAv2AttentionMetadataBuilder

        @staticmethod
        def get_kv_cache_shape(num_blocks: int, block_size: int, num_kv_heads: int,
                               head_size: int, cache_dtype_str: str = "auto") -> tuple:
            """Always the compact fp16 shape ``(nb, bs, H_kv, 72)``; the page
            accounting is switched to 144-byte slots when vLLM is present."""
            if head_size != HEAD_DIM:
                raise ValueError(f"CDA backend supports head_size={HEAD_DIM} only. "
                                 f"Got head_size={head_size}.")
            if have_vllm and not getattr(b["AttentionSpec"], "_cda_v2_patched", False):
                enable_cda_memory_saving()
            return (num_blocks, block_size, num_kv_heads, _SLOT_FP16_ELEMS_COMPACT)

        @classmethod
        def get_supported_head_sizes(cls) -> list:
            return [HEAD_DIM]

        @staticmethod
        def swap_blocks(src_kv_cache, dst_kv_cache, src_to_dst) -> None:
            dst_kv_cache[src_to_dst[:, 1]] = src_kv_cache[src_to_dst[:, 0]]

        @staticmethod
        def copy_blocks(kv_caches, src_to_dists) -> None:
            for kv_cache in kv_caches:
                kv_cache[src_to_dists[:, 1]] = kv_cache[src_to_dists[:, 0]]

    class CDAv2AttentionImpl(b["AttentionImpl"][CDAv2AttentionMetadataVLLM]):
        """Per-layer attention (``cda_attn_v2.py:616-1701``)."""
        can_return_lse_for_decode: bool = False

        def __init__(self, num_heads: int, head_size: int, scale: float,
                     num_kv_heads: int | None = None, alibi_slopes=None,
                     sliding_window: int | None = None, kv_cache_dtype: str = "auto",
                     logits_soft_cap: float | None = None,
                     attn_type: str = AttentionType.DECODER,
                     kv_sharing_target_layer_name: str | None = None) -> None:
            self.num_heads = num_heads
            self.head_size = head_size
            self.scale = float(scale)
            self.num_kv_heads = num_kv_heads or num_heads
            self.group_size = self.num_heads // self.num_kv_heads
            self.attn_type = attn_type
            if alibi_slopes is not None:
                raise NotImplementedError("CDA backend does not support ALiBi.")
            if sliding_window is not None:
                raise NotImplementedError("CDA backend does not support sliding window.")
            if attn_type != AttentionType.DECODER:
                raise NotImplementedError(f"CDA backend is DECODER-only, got {attn_type}.")
            if self.group_size not in (4, 8):
                raise NotImplementedError(
                    f"CDA supports group_size in {{4, 8}}, got group_size={self.group_size}.")

        # -- cache update ----------------------------------------------------
        def do_kv_cache_update(self, layer, key: torch.Tensor, value: torch.Tensor,
                               kv_cache: torch.Tensor, slot_mapping: torch.Tensor) -> None:
            """Encode this step's K/V (T, H_kv, 128) fp16 into their slots
            (``cda_attn_v2.py:655-677``); negative slots are skipped."""
            if kv_cache.numel() == 0:
                return

            def run():
                from sub0_amd.cda.kernels_cuda.wrappers import paged_encode_fused_cuda
                cache = _as_uint8_cache(kv_cache)
                nb, bs, hkv, width = cache.shape
                cmp_K, cmp_V = _get_compressors(cache.device)
                paged_encode_fused_cuda(key, value, slot_mapping,
                                        cache.view(nb * bs, hkv, width),
                                        cb_K=cmp_K.codebook, cb_V=cmp_V.codebook)
            _time_call("do_kv_cache_update", run)

        # -- dispatch --------------------------------------------------------
        def forward(self, layer, query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                    kv_cache: torch.Tensor, attn_metadata, output: torch.Tensor | None = None,
                    output_scale=None, output_block_scale=None) -> torch.Tensor:
            """Attention of ``query`` (T, H_q, 128) over the compressed cache
            into ``output`` (``cda_attn_v2.py:679-748``): decode when every
            request has one query token, prefill when none has, and both
            (decode rows first) for a mixed chunked-prefill batch."""
            if output is None:
                raise ValueError("CDA backend requires an output buffer.")
            if output_scale is not None or output_block_scale is not None:
                raise NotImplementedError(
                    "CDA backend does not support fused output quantization.")
            if attn_metadata is None:
                return output.fill_(0)
            kv_cache = _as_uint8_cache(kv_cache)
            if attn_metadata.dcp_world_size > 1:
                return _time_call("_forward_dcp", lambda: self._forward_decode_dcp(
                    query, kv_cache, output, attn_metadata))
            if attn_metadata.max_query_len > 1:
                md = attn_metadata
                nd = getattr(md, "num_decodes", 0)
                npf = getattr(md, "num_prefills", 0)
                nd_tok = getattr(md, "num_decode_tokens", 0)
                np_tok = getattr(md, "num_prefill_tokens", 0)
                if nd + npf != md.num_reqs or nd_tok + np_tok != md.num_actual_tokens:
                    nd, npf, nd_tok, np_tok = _split_counts_from_query_start(
                        md.query_start_loc, md.num_reqs, md.num_actual_tokens,
                        md.max_query_len)
                    md.num_decodes, md.num_prefills = nd, npf
                    md.num_decode_tokens, md.num_prefill_tokens = nd_tok, np_tok
                if nd_tok > 0 and np_tok > 0:
                    return _time_call("_forward_prefill_decode",
                                      lambda: self._forward_mixed_prefill_decode(
                                          query, key, value, output, md, kv_cache))
                return _time_call("_forward_prefill", lambda: self._forward_prefill(
                    query, key, value, output, md, kv_cache))
            return _time_call("_forward_decode", lambda: self._forward_decode(
                query, kv_cache, output, attn_metadata))

        def _forward_mixed_prefill_decode(self, query, key, value, output, attn_metadata,
                                          kv_cache):
            """Decode rows through the decode kernel, the remaining rows through
            prefill, each on its slice of the metadata
            (``cda_attn_v2.py:760-836``)."""
            md = attn_metadata
            nd, npf = md.num_decodes, md.num_prefills
            nd_tok, np_tok = md.num_decode_tokens, md.num_prefill_tokens
            if nd_tok <= 0 or np_tok <= 0:
                raise ValueError("mixed prefill/decode requires both phases")
            if key is None or value is None:
                raise ValueError("mixed prefill/decode requires key/value")
            dec = CDAv2AttentionMetadata(
                num_actual_tokens=nd_tok, num_reqs=nd, max_query_len=1,
                max_seq_len=md.max_seq_len, query_start_loc=md.query_start_loc[:nd + 1],
                seq_lens=md.seq_lens[:nd], block_table=md.block_table[:nd],
                slot_mapping=md.slot_mapping[:nd_tok], causal=md.causal,
                num_decode_tokens=nd_tok, num_decodes=nd)
            self._forward_decode(query[:nd_tok], kv_cache, output[:nd_tok], dec)
            end = nd_tok + np_tok
            pre = CDAv2AttentionMetadata(
                num_actual_tokens=np_tok, num_reqs=npf, max_query_len=md.max_query_len,
                max_seq_len=md.max_seq_len, query_start_loc=md.query_start_loc[nd:] - nd_tok,
                seq_lens=md.seq_lens[nd:nd + npf], block_table=md.block_table[nd:nd + npf],
                slot_mapping=md.slot_mapping[nd_tok:end], causal=md.causal,
                num_prefill_tokens=np_tok, num_prefills=npf)
            self._forward_prefill(query[nd_tok:end], key[nd_tok:end], value[nd_tok:end],
                                  output[nd_tok:end], pre, kv_cache)
            return output

        def _setup(self, query, kv_cache):
            """``(cb_K, cb_V, rot_fp32, rot_fp16, flat_cache, block_size)``
            (``cda_attn_v2.py:884-900``)."""
            nb, bs, hkv, width = kv_cache.shape
            cmp_K, cmp_V = _get_compressors(query.device)
            cb_K, cb_V, r32, r16 = _get_hmma_artifacts(cmp_K, cmp_V, query.device)
            return cb_K, cb_V, r32, r16, kv_cache.view(nb * bs, hkv, width), bs

        _p34_setup = _setup

        # -- prefill ---------------------------------------------------------
        def _forward_prefill(self, query, key, value, output, attn_metadata, kv_cache):
            """Causal prefill of every query row over its request's keys
            (``cda_attn_v2.py:838-882, 1330-1472``).  ``CDA_PREFILL_BACKEND``
            picks the route: ``fa2_cda_fused`` (default), ``fa2_cda_auto``,
            ``fa2_cda_direct[_v2]`` and ``fa2_cda`` run the prefill kernel over
            the compressed cache; ``fa2_rawkv``, ``fa2_cda_rawkv`` and
            ``fa2_cda_fused_rawkv`` attend to the fresh fp16 K/V of the chunk
            instead (``:1402-1441``): with a compressed prefix
            (``max_seq_len > max_query_len``) through the hybrid kernel,
            without one through plain FA2 (``fa2_rawkv``) or the fused FA2-CDA
            kernel fed from the rotated raw K/V.  The P34 ``hmma`` route is not
            built."""
            md = attn_metadata
            L = int(md.max_query_len)
            route = os.getenv("CDA_PREFILL_BACKEND", "fa2_cda_fused").lower()
            if route not in _PREFILL_FUSED + _PREFILL_UNFUSED + _PREFILL_RAWKV:
                raise NotImplementedError(
                    f"CDA_PREFILL_BACKEND={route!r} is not available in the MI355X build; "
                    f"expected one of {_PREFILL_FUSED + _PREFILL_UNFUSED + _PREFILL_RAWKV}.")
            if L <= 0:
                raise NotImplementedError("CDA prefill received an empty prefill chunk.")
            T = int(md.num_actual_tokens)
            H_q, D = self.num_heads, self.head_size
            cb_K, cb_V, r32, r16, flat, bs = _time_call(
                "prefill_setup", lambda: self._setup(query, kv_cache))
            q = query[:T]
            if q.dtype != torch.float16:
                q = _time_call("prefill_q_cast", lambda: q.to(torch.float16))
            out = _fp16_view(output, T, H_q, D)
            direct = out is not None
            if not direct:
                out = torch.empty(T, H_q, D, dtype=torch.float16, device=query.device)
            if route in _PREFILL_RAWKV:
                if key is None or value is None:
                    raise ValueError(f"{route} requires fresh prefill key/value tensors")
                k_new, v_new = key[:T], value[:T]
                if int(md.max_seq_len) > L:
                    from sub0_amd.cda.kernels_cuda.wrappers import hybrid_attn_v1
                    _time_call("prefill_hybrid_rawkv_chunked", lambda: hybrid_attn_v1(
                        q, k_new, v_new, out, flat, md.block_table,
                        cu_seqlens_q=md.query_start_loc, seq_lens=md.seq_lens,
                        cb_K=cb_K, cb_V=cb_V, rotation_fp32=r32, rotation_fp16=r16,
                        scale=self.scale, group_size=self.group_size, block_size=bs,
                        max_seq_len=int(md.max_seq_len), max_query_len=L))
                elif route == "fa2_rawkv":
                    from sub0_amd.cda.kernels_cuda.fa2_cda import fa2_raw_prefill_varlen_v1
                    _time_call("prefill_fa2_rawkv", lambda: fa2_raw_prefill_varlen_v1(
                        q, k_new, v_new, md.query_start_loc, out, group_size=self.group_size,
                        max_query_len=L, scale=self.scale, causal=True))
                else:
                    from sub0_amd.cda.kernels_cuda.fa2_cda import (
                        fa2_cda_prefill_rawkv_varlen_v1)
                    _time_call("prefill_fa2_cda_rawkv", lambda: fa2_cda_prefill_rawkv_varlen_v1(
                        q, k_new, v_new, md.query_start_loc, md.seq_lens, out,
                        rotation_fp32=r32, group_size=self.group_size, max_query_len=L,
                        max_seq_len=int(md.max_seq_len), scale=self.scale, causal=True))
            else:
                from sub0_amd.cda.kernels_cuda.fa2_cda import fa2_cda_prefill_varlen_v1
                _time_call("prefill_fa2_cda", lambda: fa2_cda_prefill_varlen_v1(
                    q, flat, md.block_table, md.query_start_loc, md.seq_lens, out,
                    cb_K=cb_K, cb_V=cb_V, rotation_fp32=r32, group_size=self.group_size,
                    block_size=bs, max_query_len=L, max_seq_len=md.max_seq_len,
                    scale=self.scale, causal=True,
                    fuse_fa2_epilogue=route in _PREFILL_FUSED))
            if not direct:
                _time_call("prefill_output_copy", lambda: _copy_out(output, out, T))
            return output

        # -- decode ----------------------------------------------------------
        def _call_decode_hmma_v1(self, q_in, kv_cache_flat, attn_metadata, out_buf, *,
                                 cb_K, cb_V, rotation_fp32, rotation_fp16, block_size):
            """One split-K decode launch (``cda_attn_v2.py:1301-1328``)."""
            from sub0_amd.cda.kernels_cuda.wrappers import decode_hmma_v1
            decode_hmma_v1(q_in, kv_cache_flat, attn_metadata.block_table,
                           attn_metadata.seq_lens, out_buf, cb_K=cb_K, cb_V=cb_V,
                           rotation_fp32=rotation_fp32, rotation_fp16=rotation_fp16,
                           group_size=self.group_size, block_size=block_size,
                           scale=self.scale, max_seq_len=attn_metadata.max_seq_len)

        def _call_dequant_fa2_decode(self, q_in, kv_cache_flat, attn_metadata, out_buf, *,
                                     cb_K, cb_V, rotation_fp32, rotation_fp16, block_size):
            """Class-(a) R2 comparator (``cda_attn_v2.py:1062-1184``): dense
            dequantised K/V, then attention over them."""
            from sub0_amd.cda.kernels_cuda.class_a import dequant_fa2_decode
            B = q_in.shape[0]
            dequant_fa2_decode(q_in, kv_cache_flat, attn_metadata.block_table[:B],
                               attn_metadata.seq_lens[:B], out_buf, cb_K=cb_K, cb_V=cb_V,
                               rotation_fp32=rotation_fp32, block_size=block_size,
                               max_seq_len=attn_metadata.max_seq_len, scale=self.scale)

        def _call_fused_dequant_fa2_decode(self, q_in, kv_cache_flat, attn_metadata, out_buf, *,
                                           cb_K, cb_V, rotation_fp32, rotation_fp16,
                                           block_size):
            """Class-(a) R1 comparator (``cda_attn_v2.py:1186-1250``): tiles of
            the compressed cache dequantised on chip inside the attention."""
            from sub0_amd.cda.kernels_cuda.class_a import fused_dequant_fa2_decode
            B = q_in.shape[0]
            fused_dequant_fa2_decode(q_in, kv_cache_flat, attn_metadata.block_table[:B],
                                     attn_metadata.seq_lens[:B], out_buf, cb_K=cb_K,
                                     cb_V=cb_V, block_size=block_size, scale=self.scale)

        def _forward_decode(self, query, kv_cache, output, attn_metadata):
            """One query token per request over the paged cache, written
            straight into ``output`` when it is an fp16 (T, H_q, D) or
            (T, H_q*D) buffer (``cda_attn_v2.py:1565-1695``).  Graph-capturable:
            no host synchronisation."""
            if kv_cache.shape[3] % 16 != 0:
                raise NotImplementedError(
                    "CDA decode requires 16-byte aligned compressed slots.")
            if _DECODE_BACKEND not in ("hmma_v1", "dequant_fa2", "fused_dequant_fa2"):
                raise NotImplementedError(
                    f"CDA_DECODE_BACKEND={_DECODE_BACKEND!r} is not a decode route; expected "
                    "hmma_v1, dequant_fa2 or fused_dequant_fa2.")
            cb_K, cb_V, r32, r16, flat, bs = _time_call(
                "decode_setup", lambda: self._setup(query, kv_cache))
            q = query.squeeze(2) if query.dim() == 4 else query
            if q.dtype != torch.float16:
                q = _time_call("decode_q_cast", lambda: q.to(torch.float16))
            T = q.shape[0]
            out = None if _USE_HMMA_V1 else _fp16_view(output, T, self.num_heads,
                                                      self.head_size)
            direct = out is not None and output.shape[0] == T
            if not direct:
                out = torch.empty_like(q)
            if _DECODE_BACKEND == "dequant_fa2":
                _time_call("decode_dequant_fa2", lambda: self._call_dequant_fa2_decode(
                    q, flat, attn_metadata, out, cb_K=cb_K, cb_V=cb_V, rotation_fp32=r32,
                    rotation_fp16=r16, block_size=bs))
            elif _DECODE_BACKEND == "fused_dequant_fa2":
                _time_call("decode_fused_dequant_fa2", lambda: self._call_fused_dequant_fa2_decode(
                    q, flat, attn_metadata, out, cb_K=cb_K, cb_V=cb_V, rotation_fp32=r32,
                    rotation_fp16=r16, block_size=bs))
            else:
                _time_call("decode_hmma", lambda: self._call_decode_hmma_v1(
                    q, flat, attn_metadata, out, cb_K=cb_K, cb_V=cb_V, rotation_fp32=r32,
                    rotation_fp16=r16, block_size=bs))
            if not direct:
                _time_call("decode_output_copy", lambda: _copy_out(output, out, T))
            return output

        def _forward_decode_dcp(self, query, kv_cache, output, attn_metadata):
            """Decode-context parallelism is not implemented (as in the
            reference, ``cda_attn_v2.py:1697-1701``)."""
            raise NotImplementedError(
                "CDA DCP decode needs a partial-attention kernel; not available.")

    _CLASSES = (CDAv2AttentionBackend, CDAv2AttentionImpl, CDAv2AttentionMetadataBuilder,
                CDAv2AttentionMetadataVLLM)
    return _CLASSES


def get_backend_classes():
    """``(Backend, Impl, MetadataBuilder, Metadata)`` (``cda_attn_v2.py:1707-1709``)."""
    return _build_backend_classes()


def register_backend(slot: str = "CDA") -> None:
    """Point vLLM's ``AttentionBackendEnum[slot]`` at this backend
    (``cda_attn_v2.py:1712-1747``).  Needs vLLM; call before building ``LLM``."""
    from sub0_amd.cda.vllm_integration import _backend_eager
    from vllm.v1.attention.backends.registry import AttentionBackendEnum
    from vllm.v1.attention.backends.registry import register_backend as _vllm_register
    try:
        target = AttentionBackendEnum[slot]
    except (KeyError, ValueError) as e:
        raise ValueError(f"slot={slot!r} is not a known AttentionBackendEnum member") from e
    _vllm_register(target, f"{_backend_eager.__name__}.CDAv2AttentionBackend")


__all__ = [
    "CDAv2AttentionMetadata",
    "enable_cda_memory_saving",
    "get_backend_classes",
    "register_backend",
    "HEAD_DIM",
]
