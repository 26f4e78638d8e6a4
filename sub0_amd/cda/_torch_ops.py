"""torch.ops registration of the MI355X CDA kernels.

Two namespaces are registered with ``torch.library`` (schemas with
``Tensor(a!)`` annotations on the outputs written in place, CUDA (= HIP)
implementations that call the C ABI of ``libcda_hip.so`` through
:mod:`sub0_amd._native`, and fake kernels so the ops trace under
``torch.compile`` / FakeTensor):

``torch.ops.cda_hip`` -- the product entry points the reference reaches
through its pybind modules (``cda/kernels_cuda/wrappers.py:115-124,
153-156``, ``fa2_cda.py:51-52, 85-95, 166-181``): ``decode``, ``encode``,
``decode_uniform_qk``, ``qk_scores_uniform4``, ``prefill``, ``prefill_hybrid``,
``paged_to_dense``, ``varlen_fwd_hadamard``, ``varlen_fwd``, ``hadamard128``.
``load_pybind_module`` routes its module functions through these ops.

``torch.ops._cda_vllm_fa2_fork_C`` -- the comparator namespace of the
reference's vLLM FA2 fork (``cda/kernels_vllm_fa2_fork/interface.py:
138-162, 234-257, 304-328, 434-461``, loaded by
``load_torch_ops_library("_cda_vllm_fa2_fork_C")``): ``dequantize_compressed_kv``,
``varlen_fwd``, ``varlen_fwd_compressed_kv``, ``varlen_fwd_compressed_kv_fused``,
with the reference's positional signatures.  They run in the rotated frame
(no Hadamard), fp16, head_dim 128, GQA 4 or 8: the compressed variants
dequantise K/V rows with ``cda_dequantize_rows`` and attend with
``cda_fa2_varlen_fwd``.  They return ``[out, softmax_lse]`` with an empty
``softmax_lse`` (the fork fills it only for ``return_softmax`` with dropout,
which inference never uses); dropout, ALiBi, sliding windows, soft-capping
and split-KV raise ``NotImplementedError``.
"""
from __future__ import annotations

import torch

from sub0_amd import _native

_libs = []


def _define(lib: torch.library.Library, schema: str, impl, fake) -> None:
    name = schema.split("(", 1)[0]
    lib.define(schema)
    lib.impl(name, impl, "CUDA")
    torch.library.register_fake(f"{lib.ns}::{name}", fake, lib=lib)


# ----------------------------------------------------------------- cda_hip --

def _decode(q, kv_cache, block_table, seq_lens, cb_k, cb_v, rot_f32, rot_f16, out,
            group_size, block_size, tile_n, max_seq_len, scale):
    _native.decode(q, kv_cache, block_table, seq_lens, cb_k, cb_v, rot_f32, rot_f16, out,
                   group_size=group_size, block_size=block_size, tile_n=tile_n,
                   max_seq_len=max_seq_len, scale=scale)


def _decode_uniform_qk(q, kv_cache, block_table, seq_lens, cb_k, cb_v, rot_f32, out,
                       group_size, block_size, tile_n, max_seq_len, scale):
    _native.decode(q, kv_cache, block_table, seq_lens, cb_k, cb_v, rot_f32, None, out,
                   group_size=group_size, block_size=block_size, tile_n=tile_n,
                   max_seq_len=max_seq_len, scale=scale, uniform_qk=True)


def _qk_scores(q_rot, k_idx, k_norm, out, group_size, scale, causal, q_offset, key_start,
               key_end):
    _native.qk_scores_uniform4(q_rot, k_idx, k_norm, out, group_size=group_size, scale=scale,
                               causal=causal, q_offset=q_offset, key_start=key_start,
                               key_end=key_end)


def _encode(k, v, slot_mapping, flat_cache, cb_k, cb_v):
    _native.paged_encode(k, v, slot_mapping, flat_cache, cb_k, cb_v)


def _prefill(q, kv_cache, block_table, cu_seqlens_q, seq_lens, cb_k, cb_v, out, block_size,
             max_query_len, scale, max_seq_len):
    _native.prefill_paged(q, kv_cache, block_table, cu_seqlens_q, seq_lens, cb_k, cb_v, out,
                          block_size=block_size, max_query_len=max_query_len, scale=scale,
                          max_seq_len=None if max_seq_len < 0 else max_seq_len)


def _prefill_hybrid(q, k_new, v_new, kv_cache, block_table, cu_seqlens_q, seq_lens, cb_k,
                    cb_v, out, block_size, max_query_len, max_seq_len, scale):
    _native.prefill_hybrid(q, k_new, v_new, kv_cache, block_table, cu_seqlens_q, seq_lens, cb_k,
                           cb_v, out, block_size=block_size, max_query_len=max_query_len,
                           max_seq_len=max_seq_len, scale=scale)


def _varlen_fwd_plain(q, k, v, out, cu_q, cu_k, seqused_k, max_q, scale, causal):
    _native.fa2_varlen_fwd(q, k, v, out, cu_q, cu_k, seqused_k, max_q, scale, causal)


def _paged_to_dense(kv_cache, block_table, seq_lens, cb_k, cb_v, block_size, max_seq_len):
    return _native.paged_to_dense(kv_cache, block_table, seq_lens, cb_k, cb_v,
                                  block_size=block_size, max_seq_len=max_seq_len)


def _paged_to_dense_fake(kv_cache, block_table, seq_lens, cb_k, cb_v, block_size, max_seq_len):
    shape = (seq_lens.shape[0] * max_seq_len, kv_cache.shape[1], 128)
    k = kv_cache.new_empty(shape, dtype=torch.float16)
    return k, torch.empty_like(k)


def _varlen_fwd_hadamard(q, k_rot, v_rot, out, cu_q, cu_k, seqused_k, max_q, max_k, scale):
    _native.fa2_varlen_fwd_hadamard(q, k_rot, v_rot, out, cu_q, cu_k, seqused_k, max_q, max_k,
                                    scale)


def _hadamard128(x, y, scale):
    _native.hadamard128(x, y, scale)


def _nothing(*args):
    return None


_cda = torch.library.Library("cda_hip", "DEF")
_libs.append(_cda)
_define(_cda, "decode(Tensor q, Tensor kv_cache, Tensor block_table, Tensor seq_lens, "
              "Tensor cb_k, Tensor cb_v, Tensor rot_f32, Tensor rot_f16, Tensor(a!) out, "
              "int group_size, int block_size, int tile_n, int max_seq_len, float scale) -> ()",
        _decode, _nothing)
_define(_cda, "decode_uniform_qk(Tensor q, Tensor kv_cache, Tensor block_table, "
              "Tensor seq_lens, Tensor cb_k, Tensor cb_v, Tensor rot_f32, Tensor(a!) out, "
              "int group_size, int block_size, int tile_n, int max_seq_len, float scale) -> ()",
        _decode_uniform_qk, _nothing)
_define(_cda, "qk_scores_uniform4(Tensor q_rot, Tensor k_idx, Tensor k_norm, Tensor(a!) out, "
              "int group_size, float scale, bool causal, int q_offset, int key_start, "
              "int key_end) -> ()", _qk_scores, _nothing)
_define(_cda, "encode(Tensor k, Tensor v, Tensor slot_mapping, Tensor(a!) flat_cache, "
              "Tensor cb_k, Tensor cb_v) -> ()", _encode, _nothing)
_define(_cda, "prefill(Tensor q, Tensor kv_cache, Tensor block_table, Tensor cu_seqlens_q, "
              "Tensor seq_lens, Tensor cb_k, Tensor cb_v, Tensor(a!) out, int block_size, "
              "int max_query_len, float scale, int max_seq_len=-1) -> ()", _prefill, _nothing)
_define(_cda, "prefill_hybrid(Tensor q, Tensor k_new, Tensor v_new, Tensor kv_cache, "
              "Tensor block_table, Tensor cu_seqlens_q, Tensor seq_lens, Tensor cb_k, "
              "Tensor cb_v, Tensor(a!) out, int block_size, int max_query_len, "
              "int max_seq_len, float scale) -> ()", _prefill_hybrid, _nothing)
_define(_cda, "varlen_fwd(Tensor q, Tensor k, Tensor v, Tensor(a!) out, Tensor cu_seqlens_q, "
              "Tensor cu_seqlens_k, Tensor seqused_k, int max_seqlen_q, float scale, "
              "bool causal) -> ()", _varlen_fwd_plain, _nothing)
_define(_cda, "paged_to_dense(Tensor kv_cache, Tensor block_table, Tensor seq_lens, "
              "Tensor cb_k, Tensor cb_v, int block_size, int max_seq_len) -> (Tensor, Tensor)",
        _paged_to_dense, _paged_to_dense_fake)
_define(_cda, "varlen_fwd_hadamard(Tensor q, Tensor k_rot, Tensor v_rot, Tensor(a!) out, "
              "Tensor cu_seqlens_q, Tensor cu_seqlens_k, Tensor seqused_k, int max_seqlen_q, "
              "int max_seqlen_k, float scale) -> ()", _varlen_fwd_hadamard, _nothing)
_define(_cda, "hadamard128(Tensor x, Tensor(a!) y, float scale) -> ()", _hadamard128, _nothing)


# ------------------------------------------------- _cda_vllm_fa2_fork_C --

def _unsupported(p_dropout, window_left, window_right, softcap, num_splits, alibi=None,
                 block_table=None):
    if p_dropout != 0.0:
        raise NotImplementedError("inference only: p_dropout must be 0")
    if window_left != -1 or window_right != -1:
        raise NotImplementedError("sliding windows are not supported")
    if softcap != 0.0:
        raise NotImplementedError("soft-capping is not supported")
    if num_splits > 1:
        raise NotImplementedError("split-KV is not supported")
    if alibi is not None:
        raise NotImplementedError("ALiBi is not supported")
    if block_table is not None:
        raise NotImplementedError("paged dense K/V is not supported by varlen_fwd")


def _seqused(cu_k, seqused_k):
    if seqused_k is not None:
        return seqused_k.to(torch.int32).contiguous()
    return (cu_k[1:] - cu_k[:-1]).to(torch.int32).contiguous()


def _attend(q, k, v, out, cu_q, cu_k, seqused, max_q, scale, causal):
    if out is None:
        out = torch.empty_like(q)
    _native.fa2_varlen_fwd(q.contiguous(), k.contiguous(), v.contiguous(), out,
                           cu_q.to(torch.int32).contiguous(), cu_k.to(torch.int32).contiguous(),
                           seqused, int(max_q), float(scale), bool(causal))
    return [out, q.new_empty((0,), dtype=torch.float32)]


def _fork_dequant(k_idx, k_norm, v_idx, v_norm, cb_k, cb_v):
    k = _native.dequantize_rows(k_idx, k_norm, cb_k.float())
    v = _native.dequantize_rows(v_idx, v_norm, cb_v.float())
    return k, v


def _fork_dequant_fake(k_idx, k_norm, v_idx, v_norm, cb_k, cb_v):
    shape = (k_idx.shape[0], k_idx.shape[1], 128)
    return (k_idx.new_empty(shape, dtype=torch.float16),
            v_idx.new_empty(shape, dtype=torch.float16))


def _fork_varlen_fwd(q, k, v, out, cu_q, cu_k, seqused_k, leftpad_k, block_table, alibi, max_q,
                     max_k, p_dropout, scale, zero_tensors, causal, wl, wr, softcap,
                     return_softmax, num_splits, gen):
    _unsupported(p_dropout, wl, wr, softcap, num_splits, alibi, block_table)
    if leftpad_k is not None:
        raise NotImplementedError("leftpad_k is not supported")
    return _attend(q, k, v, out, cu_q, cu_k, _seqused(cu_k, seqused_k), max_q, scale, causal)


def _fork_varlen_compressed(q, k_idx, k_norm, v_idx, v_norm, cb_k, cb_v, out, cu_q, cu_k, alibi,
                            max_q, max_k, p_dropout, scale, zero_tensors, causal, wl, wr,
                            softcap, return_softmax, num_splits, gen):
    _unsupported(p_dropout, wl, wr, softcap, num_splits, alibi)
    k, v = _fork_dequant(k_idx, k_norm, v_idx, v_norm, cb_k, cb_v)
    return _attend(q, k, v, out, cu_q, cu_k, _seqused(cu_k, None), max_q, scale, causal)


def _fork_varlen_compressed_fused(q, k_idx, k_norm, v_idx, v_norm, cb_k, cb_v, out, cu_q, cu_k,
                                  seqused_k, block_table, alibi, max_q, max_k, p_dropout, scale,
                                  zero_tensors, causal, wl, wr, softcap, return_softmax,
                                  num_splits, uniform_codebook, gen):
    _unsupported(p_dropout, wl, wr, softcap, num_splits, alibi)
    if block_table is None:
        k, v = _fork_dequant(k_idx, k_norm, v_idx, v_norm, cb_k, cb_v)
        return _attend(q, k, v, out, cu_q, cu_k, _seqused(cu_k, seqused_k), max_q, scale, causal)
    # Paged pools (num_blocks, block_size, H_kv, D/2) + (num_blocks, block_size, H_kv):
    # gather each sequence's tokens into dense rows b * max_k + t, then attend.
    nb, bs, H, cbytes = k_idx.shape
    bt = block_table.to(torch.int32).contiguous()
    sl = seqused_k.to(torch.int32).contiguous()
    kw = dict(block_table=bt, seq_lens=sl, block_size=bs, max_seq_len=int(max_k))
    k = _native.dequantize_rows(k_idx.reshape(nb * bs, H, cbytes), k_norm.reshape(nb * bs, H),
                                cb_k.float(), **kw)
    v = _native.dequantize_rows(v_idx.reshape(nb * bs, H, cbytes), v_norm.reshape(nb * bs, H),
                                cb_v.float(), **kw)
    B = sl.numel()
    cu_dense = torch.arange(B + 1, dtype=torch.int32, device=q.device) * int(max_k)
    return _attend(q, k, v, out, cu_q, cu_dense, sl, max_q, scale, causal)


def _fork_fake(q, *args):
    out = args[6] if len(args) > 6 and isinstance(args[6], torch.Tensor) else None
    return [torch.empty_like(q) if out is None else out, q.new_empty((0,), dtype=torch.float32)]


def _fork_varlen_fwd_fake(q, k, v, out, *rest):
    return [torch.empty_like(q) if out is None else out, q.new_empty((0,), dtype=torch.float32)]


_TAIL = ("int max_seqlen_q, int max_seqlen_k, float p_dropout, float softmax_scale, "
         "bool zero_tensors, bool is_causal, int window_size_left, int window_size_right, "
         "float softcap, bool return_softmax, int num_splits")

_fork = torch.library.Library("_cda_vllm_fa2_fork_C", "DEF")
_libs.append(_fork)
_define(_fork, "dequantize_compressed_kv(Tensor k_idx, Tensor k_norm, Tensor v_idx, "
               "Tensor v_norm, Tensor cb_k, Tensor cb_v) -> (Tensor, Tensor)",
        _fork_dequant, _fork_dequant_fake)
_define(_fork, "varlen_fwd(Tensor q, Tensor k, Tensor v, Tensor(a!)? out, Tensor cu_seqlens_q, "
               "Tensor cu_seqlens_k, Tensor? seqused_k, Tensor? leftpad_k, Tensor? block_table, "
               "Tensor? alibi_slopes, " + _TAIL + ", Generator? gen) -> Tensor[]",
        _fork_varlen_fwd, _fork_varlen_fwd_fake)
_define(_fork, "varlen_fwd_compressed_kv(Tensor q, Tensor k_idx, Tensor k_norm, Tensor v_idx, "
               "Tensor v_norm, Tensor cb_k, Tensor cb_v, Tensor(a!)? out, Tensor cu_seqlens_q, "
               "Tensor cu_seqlens_k, Tensor? alibi_slopes, " + _TAIL +
               ", Generator? gen) -> Tensor[]",
        _fork_varlen_compressed, _fork_fake)
_define(_fork, "varlen_fwd_compressed_kv_fused(Tensor q, Tensor k_idx, Tensor k_norm, "
               "Tensor v_idx, Tensor v_norm, Tensor cb_k, Tensor cb_v, Tensor(a!)? out, "
               "Tensor cu_seqlens_q, Tensor cu_seqlens_k, Tensor? seqused_k, "
               "Tensor? block_table, Tensor? alibi_slopes, " + _TAIL +
               ", bool uniform_codebook, Generator? gen) -> Tensor[]",
        _fork_varlen_compressed_fused, _fork_fake)

NAMESPACES = ("cda_hip", "_cda_vllm_fa2_fork_C")
