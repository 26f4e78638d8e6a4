"""Seeded CDA test cases shared by the GPU parity tests (uses the CPU checker)."""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from oracle import cda_oracle as O
from oracle import synth

D = 128


@dataclass
class DecodeCase:
    q: np.ndarray            # (B, H_q, 128) fp16
    cache: np.ndarray        # (slots, H_kv, slot_bytes) uint8
    block_table: np.ndarray  # (B, W) int32
    seq_lens: np.ndarray     # (B,) int32
    cb_k: np.ndarray
    cb_v: np.ndarray
    R: np.ndarray
    H_kv: int
    block_size: int
    expected: np.ndarray     # oracle output (B, H_q, 128) fp16


def _ramp(k, k_ramp):
    """K rows scaled by 1 + k_ramp * t / n along the key axis (axis 2): scores
    that grow along the sequence, so a running max keeps moving."""
    if not k_ramp:
        return k
    n = k.shape[2]
    f = 1.0 + k_ramp * np.arange(n, dtype=np.float32) / max(1, n)
    return (k.astype(np.float32) * f[None, None, :, None]).astype(np.float16)


def make_decode_case(seed, seq_lens, *, H_kv=8, gs=4, block_size=16, cb=None, extra_blocks=3,
                     scale=None, fill=0, cb_v=None, k_ramp=0.0):
    """Encode seeded K/V per sequence with the checker, scatter into a paged
    cache through a permuted block table, and compute the checker's output."""
    seq_lens = np.asarray(seq_lens, dtype=np.int32)
    B = len(seq_lens)
    H_q = H_kv * gs
    if cb is None:
        cb = synth_cb()
    if cb_v is None:
        cb_v = cb
    nmax = max(1, int(seq_lens.max()))
    W = (nmax + block_size - 1) // block_size + extra_blocks
    bt = synth.permuted_block_table(seed, B, W)
    k = _ramp(synth.kv_with_outliers(seed, (B, H_kv, nmax, D)), k_ramp)
    v = synth.normal_f16(seed + 1, (B, H_kv, nmax, D))
    q = synth.normal_f16(seed + 2, (B, H_q, D))
    kp, kn, _ = O.encode(k, cb)
    vp, vn, _ = O.encode(v, cb_v)
    cache = O.build_paged_cache(kp, kn, vp, vn, bt, block_size, cb.size,
                                num_blocks=B * W, fill=fill)
    R = O.hadamard128()
    exp = O.decode_paged(q, cache, bt, seq_lens, cb, cb_v, R, H_kv=H_kv,
                         block_size=block_size, scale=scale)
    return DecodeCase(q, cache, bt, seq_lens, cb, cb_v, R, H_kv, block_size, exp)


_CB = None


def synth_cb():
    global _CB
    if _CB is None:
        from pathlib import Path
        _CB = np.load(Path(__file__).parent / "golden" / "codebooks.npz")["lloyd_beta16"]
    return _CB


@dataclass
class PrefillCase:
    q: np.ndarray            # (T, H_q, 128) fp16, T = sum(seq_q)
    cu_q: np.ndarray         # (B+1,) int32
    cache: np.ndarray
    block_table: np.ndarray
    seq_k: np.ndarray        # (B,) int32 key lengths
    cb: np.ndarray
    H_kv: int
    block_size: int
    expected: np.ndarray     # oracle output (T, H_q, 128) fp16
    cb_v: np.ndarray = None  # V codebook when it differs from cb


def make_prefill_case(seed, seq_q, seq_k, *, H_kv=8, gs=4, block_size=16, scale=None, fill=0,
                      cb_v=None, k_ramp=0.0):
    """Seeded K/V for each sequence's seq_k keys (encoded by the checker into a
    paged cache), queries for its last seq_q positions, and the checker's
    causal prefill output."""
    seq_q = np.asarray(seq_q, dtype=np.int32)
    seq_k = np.asarray(seq_k, dtype=np.int32)
    B = len(seq_q)
    H_q = H_kv * gs
    cb = synth_cb()
    nmax = max(1, int(seq_k.max()))
    W = (nmax + block_size - 1) // block_size + 1
    bt = synth.permuted_block_table(seed, B, W)
    k = _ramp(synth.kv_with_outliers(seed, (B, H_kv, nmax, D)), k_ramp)
    v = synth.normal_f16(seed + 1, (B, H_kv, nmax, D))
    cbv = cb if cb_v is None else np.asarray(cb_v, dtype=np.float32)
    kp, kn, _ = O.encode(k, cb)
    vp, vn, _ = O.encode(v, cbv)
    cache = O.build_paged_cache(kp, kn, vp, vn, bt, block_size, cb.size,
                                num_blocks=B * W, fill=fill)
    cu = np.concatenate([[0], np.cumsum(seq_q)]).astype(np.int32)
    q = synth.normal_f16(seed + 2, (int(cu[-1]), H_q, D))
    R = O.hadamard128()
    exp = O.prefill_paged(q, cu, cache, bt, seq_k, cb, cbv, R, H_kv=H_kv,
                          block_size=block_size, scale=scale)
    return PrefillCase(q, cu, cache, bt, seq_k, cb, H_kv, block_size, exp, cb_v)


@dataclass
class HybridCase:
    q: np.ndarray            # (T, H_q, 128) fp16
    k_new: np.ndarray        # (T, H_kv, 128) fp16, the chunk's raw K
    v_new: np.ndarray
    cu_q: np.ndarray
    cache: np.ndarray        # all seq_k keys of each sequence, encoded
    block_table: np.ndarray
    seq_k: np.ndarray
    cb: np.ndarray
    H_kv: int
    block_size: int
    k_enc: tuple             # (packed, norm) of K per sequence (B, H_kv, nmax, ...)
    expected: np.ndarray     # checker output (T, H_q, 128) fp16


def make_hybrid_case(seed, seq_q, seq_k, *, H_kv=8, gs=4, block_size=16, scale=None):
    """Chunked prefill: every sequence's seq_k keys encoded into the paged
    cache (as the KV update does before attention), its last seq_q keys also
    given raw as the chunk's K/V, and the checker's hybrid output."""
    seq_q = np.asarray(seq_q, dtype=np.int32)
    seq_k = np.asarray(seq_k, dtype=np.int32)
    B = len(seq_q)
    H_q = H_kv * gs
    cb = synth_cb()
    nmax = max(1, int(seq_k.max()))
    W = (nmax + block_size - 1) // block_size + 1
    bt = synth.permuted_block_table(seed, B, W)
    k = synth.kv_with_outliers(seed, (B, H_kv, nmax, D))
    v = synth.normal_f16(seed + 1, (B, H_kv, nmax, D))
    kp, kn, _ = O.encode(k, cb)
    vp, vn, _ = O.encode(v, cb)
    cache = O.build_paged_cache(kp, kn, vp, vn, bt, block_size, cb.size, num_blocks=B * W)
    cu = np.concatenate([[0], np.cumsum(seq_q)]).astype(np.int32)
    T = int(cu[-1])
    q = synth.normal_f16(seed + 2, (T, H_q, D))
    k_new = np.zeros((T, H_kv, D), np.float16)
    v_new = np.zeros((T, H_kv, D), np.float16)
    for b in range(B):
        n, past = int(seq_q[b]), int(seq_k[b] - seq_q[b])
        k_new[cu[b]:cu[b + 1]] = k[b, :, past:past + n].transpose(1, 0, 2)
        v_new[cu[b]:cu[b + 1]] = v[b, :, past:past + n].transpose(1, 0, 2)
    exp = O.hybrid_prefill(q, cu, k_new, v_new, cache, bt, seq_k, cb, cb, O.hadamard128(),
                           H_kv=H_kv, block_size=block_size, scale=scale)
    return HybridCase(q, k_new, v_new, cu, cache, bt, seq_k, cb, H_kv, block_size, (kp, kn), exp)


def raw_causal_attention(q, cu_q, k, v, scale=None):
    """Plain causal varlen attention of fp16 q (T, H_q, 128) over the
    sequences' own fp16 k, v (T, H_kv, 128), in float64, fp16 out: the
    reference's no-prefix FA2 route (fa2_cda.py:373-460) has no rotation."""
    T, H_q, _ = q.shape
    gs = H_q // k.shape[1]
    s = 1.0 / np.sqrt(D) if scale is None else scale
    out = np.zeros(q.shape, np.float16)
    for b in range(len(cu_q) - 1):
        q0, q1 = int(cu_q[b]), int(cu_q[b + 1])
        n = q1 - q0
        vis = np.arange(n)[None, :] <= np.arange(n)[:, None]
        for hq in range(H_q):
            sc = q[q0:q1, hq].astype(np.float64) @ k[q0:q1, hq // gs].astype(np.float64).T * s
            sc = np.where(vis, sc, -np.inf)
            p = np.exp(sc - sc.max(1, keepdims=True))
            out[q0:q1, hq] = ((p @ v[q0:q1, hq // gs].astype(np.float64))
                              / p.sum(1, keepdims=True)).astype(np.float16)
    return out
