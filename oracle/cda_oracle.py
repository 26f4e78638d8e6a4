"""numpy/ctypes front end of the CPU checker (test infrastructure only).

Wraps ``oracle/_build/libcda_oracle.so`` (built from ``cda_oracle.c`` by
``oracle/Makefile``) and adds the pure-numpy pieces of the reference that
need no arithmetic contract:

* ``pack_4bit``/``unpack_4bit``/``pack_2bit``/``unpack_2bit``
  (``cda/algorithm/compression.py:163-188, 375-397``);
* ``uniform_centroids`` (``compression.py:75-83``);
* ``merge_partials`` (``cda/algorithm/attention.py:239-272``);
* ``hybrid_prefill``: chunked prefill over a compressed prefix plus the
  chunk's raw K/V, merged by ``merge_partials`` (the contract of
  ``cda/kernels_cuda/vllm_integration/cda_attn_v2.py:1023-1060``);
* ``build_paged_cache``: scatters encoded rows into the paged slot layout of
  ``cda/kernels_cuda/vllm_integration/cda_attn_v2.py:20-27`` (K codes | V codes
  | K norm fp32 | V norm fp32 | pad).

Only tests/, ``__graft_entry__.smoke()`` and bench.py's CPU-baseline leg may
import this module.
"""
from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "_build" / "libcda_oracle.so"
D = 128

_lib = None


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.is_file():
            build()
        L = ctypes.CDLL(str(LIB_PATH))
        P = ctypes.c_void_p
        i64, i32, f32 = ctypes.c_int64, ctypes.c_int, ctypes.c_float
        L.cda_oracle_encode_rows.argtypes = [P, i64, P, i32, P, P, P]
        L.cda_oracle_quantize.argtypes = [P, i64, P, i32, P]
        L.cda_oracle_decode_rows.argtypes = [P, P, i64, P, i32, P]
        L.cda_oracle_hadamard128.argtypes = [P]
        L.cda_oracle_f64_to_f16.argtypes = [ctypes.c_double]
        L.cda_oracle_f64_to_f16.restype = ctypes.c_uint16
        L.cda_oracle_decode_paged.argtypes = [P, P, i32, i32, i32, P, i32, P, i32, i32, i32,
                                              P, P, P, f32, i32, P]
        L.cda_oracle_decode_partial.argtypes = [P, P, i32, i32, i32, P, i32, P, i32, i32, i32,
                                                P, P, f32, i32, i32, P, P, P]
        L.cda_oracle_prefill_paged.argtypes = [P, P, P, i32, i32, i32, P, i32, P, i32, i32, i32,
                                               P, P, P, f32, P]
        L.cda_oracle_set_threads.argtypes = [i32]
        _lib = L
    return _lib


def _p(a: np.ndarray):
    assert a.flags.c_contiguous
    return a.ctypes.data_as(ctypes.c_void_p)


def set_threads(n: int) -> None:
    lib().cda_oracle_set_threads(int(n))


# ------------------------------------------------------------------ tables --

def hadamard128() -> np.ndarray:
    H = np.empty((D, D), dtype=np.float32)
    lib().cda_oracle_hadamard128(_p(H))
    return H


def uniform_centroids(L: int) -> np.ndarray:
    """compression.py:75-83: midpoints of linspace(-1, 1, L+1) in fp32."""
    edges = np.linspace(-1.0, 1.0, L + 1, dtype=np.float32)
    return ((edges[:-1] + edges[1:]) * np.float32(0.5)).astype(np.float32)


# ----------------------------------------------------------------- packing --

def pack_4bit(idx: np.ndarray) -> np.ndarray:
    idx = idx.astype(np.uint8)
    return ((idx[..., 0::2] << 4) | idx[..., 1::2]).astype(np.uint8)


def unpack_4bit(p: np.ndarray) -> np.ndarray:
    return np.stack([(p >> 4) & 0xF, p & 0xF], axis=-1).reshape(*p.shape[:-1], p.shape[-1] * 2)


def pack_2bit(idx: np.ndarray) -> np.ndarray:
    idx = idx.astype(np.uint8)
    return ((idx[..., 0::4] << 6) | (idx[..., 1::4] << 4) | (idx[..., 2::4] << 2)
            | idx[..., 3::4]).astype(np.uint8)


def unpack_2bit(p: np.ndarray) -> np.ndarray:
    return np.stack([(p >> 6) & 3, (p >> 4) & 3, (p >> 2) & 3, p & 3],
                    axis=-1).reshape(*p.shape[:-1], p.shape[-1] * 4)


# ------------------------------------------------------------ encode/decode --

def quantize_unit(x: np.ndarray, cb: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    cb = np.ascontiguousarray(cb, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint8)
    lib().cda_oracle_quantize(_p(x), x.size, _p(cb), cb.size, _p(out))
    return out


def encode(x: np.ndarray, cb: np.ndarray):
    """Compressor.encode (compression.py:315-335) on (..., 128) fp16 rows.

    Returns (packed uint8 (..., 128*bits/8), norm fp32 (...), x_rot fp16 (..., 128)).
    """
    x = np.ascontiguousarray(x, dtype=np.float16)
    cb = np.ascontiguousarray(cb, dtype=np.float32)
    L = cb.size
    bits = 4 if L == 16 else 2
    rows = x.size // D
    packed = np.empty((rows, D * bits // 8), dtype=np.uint8)
    norm = np.empty(rows, dtype=np.float32)
    xrot = np.empty((rows, D), dtype=np.uint16)
    lib().cda_oracle_encode_rows(_p(x.view(np.uint16)), rows, _p(cb), L, _p(packed), _p(norm),
                                 _p(xrot))
    lead = x.shape[:-1]
    return (packed.reshape(*lead, -1), norm.reshape(lead),
            xrot.view(np.float16).reshape(*lead, D))


def decode_rotated(packed: np.ndarray, norm: np.ndarray, cb: np.ndarray) -> np.ndarray:
    """Compressor.decode(rotated=True) (compression.py:337-361): fp16(cb[idx]*norm)."""
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    norm = np.ascontiguousarray(norm, dtype=np.float32)
    cb = np.ascontiguousarray(cb, dtype=np.float32)
    rows = norm.size
    out = np.empty((rows, D), dtype=np.uint16)
    lib().cda_oracle_decode_rows(_p(packed), _p(norm), rows, _p(cb), cb.size, _p(out))
    return out.view(np.float16).reshape(*norm.shape, D)


# ------------------------------------------------------------- paged cache --

def slot_layout(L: int, slot_bytes: int | None = None, Lv: int | None = None):
    """(code bytes per role, slot bytes).  K4V4: 64, 144 (cda_attn_v2.py:52-60);
    K2V2: 32, 80; K4V2 (Lv = 4): 64, 104 (the legacy layout, cda_attn_v2.py:29,
    K codes | V codes | K norm | V norm with no padding)."""
    kb = D * (4 if L == 16 else 2) // 8
    if Lv is not None and Lv != L:
        kbv = D * (4 if Lv == 16 else 2) // 8
        return kb, (slot_bytes if slot_bytes else kb + kbv + 8)
    data = 2 * kb + 8
    return kb, (slot_bytes if slot_bytes else (data + 15) // 16 * 16)


def _levels_arg(cbK, cbV):
    """Level argument of the C paged functions: K size, V size in bits 8..15."""
    return cbK.size if cbV.size == cbK.size else cbK.size | (cbV.size << 8)


def build_paged_cache(k_idx, k_norm, v_idx, v_norm, block_table, block_size, L,
                      num_blocks=None, slot_bytes=None, fill=0, Lv=None):
    """Scatter (B, H_kv, N, kb)/(B, H_kv, N) encodings into a
    (num_blocks*block_size, H_kv, slot_bytes) uint8 cache through block_table."""
    B, H_kv, N, kb = k_idx.shape
    kb2, sb = slot_layout(L, slot_bytes, Lv)
    assert kb == kb2
    kbv = v_idx.shape[-1]
    if num_blocks is None:
        num_blocks = int(block_table.max()) + 1
    cache = np.full((num_blocks * block_size, H_kv, sb), fill, dtype=np.uint8)
    t = np.arange(N)
    for b in range(B):
        slots = block_table[b, t // block_size].astype(np.int64) * block_size + t % block_size
        cache[slots, :, 0:kb] = k_idx[b].transpose(1, 0, 2)
        cache[slots, :, kb:kb + kbv] = v_idx[b].transpose(1, 0, 2)
        cache[slots, :, kb + kbv:kb + kbv + 4] = (
            np.ascontiguousarray(k_norm[b].T.astype(np.float32)).view(np.uint8).reshape(N, H_kv, 4))
        cache[slots, :, kb + kbv + 4:kb + kbv + 8] = (
            np.ascontiguousarray(v_norm[b].T.astype(np.float32)).view(np.uint8).reshape(N, H_kv, 4))
    return cache


def decode_paged(q, cache, block_table, seq_lens, cbK, cbV, R, *, H_kv, block_size,
                 scale=None, rotated_io=False):
    """attention_compressed (attention.py:426-482) for M_q=1 over a paged cache.

    q: (B, H_q, 128) fp16.  Returns (B, H_q, 128) fp16."""
    q = np.ascontiguousarray(q, dtype=np.float16)
    B, H_q, _ = q.shape
    cache = np.ascontiguousarray(cache, dtype=np.uint8)
    bt = np.ascontiguousarray(block_table, dtype=np.int32)
    sl = np.ascontiguousarray(seq_lens, dtype=np.int32)
    cbK = np.ascontiguousarray(cbK, dtype=np.float32)
    cbV = np.ascontiguousarray(cbV, dtype=np.float32)
    R = np.ascontiguousarray(R, dtype=np.float32)
    if scale is None:
        scale = 1.0 / np.sqrt(D)
    out = np.empty((B, H_q, D), dtype=np.uint16)
    lib().cda_oracle_decode_paged(_p(q.view(np.uint16)), _p(cache), H_kv, cache.shape[-1],
                                  _levels_arg(cbK, cbV), _p(bt), bt.shape[1], _p(sl), B, H_q, block_size,
                                  _p(cbK), _p(cbV), _p(R), float(scale), int(rotated_io),
                                  _p(out))
    return out.view(np.float16)


def decode_partial(q_rot, cache, block_table, seq_lens, cbK, cbV, *, H_kv, block_size,
                   k0, k1, scale=None):
    """Split-K partial (O_unnorm, m, l) over keys [k0, k1) (attention.py:190-236)."""
    q_rot = np.ascontiguousarray(q_rot, dtype=np.float16)
    B, H_q, _ = q_rot.shape
    cache = np.ascontiguousarray(cache, dtype=np.uint8)
    bt = np.ascontiguousarray(block_table, dtype=np.int32)
    sl = np.ascontiguousarray(seq_lens, dtype=np.int32)
    cbK = np.ascontiguousarray(cbK, dtype=np.float32)
    cbV = np.ascontiguousarray(cbV, dtype=np.float32)
    if scale is None:
        scale = 1.0 / np.sqrt(D)
    o = np.empty((B, H_q, D), dtype=np.float32)
    m = np.empty((B, H_q), dtype=np.float32)
    l = np.empty((B, H_q), dtype=np.float32)
    lib().cda_oracle_decode_partial(_p(q_rot.view(np.uint16)), _p(cache), H_kv, cache.shape[-1],
                                    _levels_arg(cbK, cbV), _p(bt), bt.shape[1], _p(sl), B, H_q, block_size,
                                    _p(cbK), _p(cbV), float(scale), int(k0), int(k1),
                                    _p(o), _p(m), _p(l))
    return o, m, l


def prefill_paged(q, cu_q, cache, block_table, seq_lens, cbK, cbV, R, *, H_kv, block_size,
                  scale=None):
    """Causal varlen prefill (attention.py:60-93, mask :46-57) over a paged cache."""
    q = np.ascontiguousarray(q, dtype=np.float16)
    T, H_q, _ = q.shape
    cu = np.ascontiguousarray(cu_q, dtype=np.int32)
    cache = np.ascontiguousarray(cache, dtype=np.uint8)
    bt = np.ascontiguousarray(block_table, dtype=np.int32)
    sl = np.ascontiguousarray(seq_lens, dtype=np.int32)
    cbK = np.ascontiguousarray(cbK, dtype=np.float32)
    cbV = np.ascontiguousarray(cbV, dtype=np.float32)
    R = np.ascontiguousarray(R, dtype=np.float32)
    if scale is None:
        scale = 1.0 / np.sqrt(D)
    out = np.empty((T, H_q, D), dtype=np.uint16)
    lib().cda_oracle_prefill_paged(_p(q.view(np.uint16)), _p(cu), _p(cache), H_kv,
                                   cache.shape[-1], _levels_arg(cbK, cbV), _p(bt), bt.shape[1], _p(sl),
                                   len(cu) - 1, H_q, block_size, _p(cbK), _p(cbV), _p(R),
                                   float(scale), _p(out))
    return out.view(np.float16)


def merge_partials(partials):
    """attention.py:239-272: online-softmax merge, NaN corrections -> 0, clamp 1e-30."""
    if not partials:
        raise ValueError("no partials to merge")
    Os = np.stack([p[0] for p in partials]).astype(np.float64)
    ms = np.stack([p[1] for p in partials]).astype(np.float64)
    ls = np.stack([p[2] for p in partials]).astype(np.float64)
    mg = ms.max(axis=0)
    with np.errstate(invalid="ignore"):
        corr = np.exp(ms - mg[None])
    corr = np.where(np.isnan(corr), 0.0, corr)
    lg = (ls * corr).sum(axis=0)
    O = (Os * corr[..., None]).sum(axis=0) / np.maximum(lg, 1e-30)[..., None]
    return O.astype(np.float16)


def paged_rows(cache, block_table, b, n, cbK, cbV, *, H_kv, block_size):
    """Rotated-frame fp16 K, V rows (H_kv, n, 128) of sequence b's first n
    keys, decoded from the paged cache (compression.py:337-361)."""
    cbK = np.asarray(cbK, dtype=np.float32)
    cbV = np.asarray(cbV, dtype=np.float32)
    kb, _ = slot_layout(cbK.size)
    kbv = slot_layout(cbV.size)[0]
    t = np.arange(n)
    rows = block_table[b, t // block_size].astype(np.int64) * block_size + t % block_size
    slots = cache[rows]                                          # (n, H_kv, slot)
    kn = np.ascontiguousarray(slots[:, :, kb + kbv:kb + kbv + 4]).view(np.float32)[..., 0]
    vn = np.ascontiguousarray(slots[:, :, kb + kbv + 4:kb + kbv + 8]).view(np.float32)[..., 0]
    k = decode_rotated(np.ascontiguousarray(slots[:, :, :kb].transpose(1, 0, 2)),
                       np.ascontiguousarray(kn.T), cbK)
    v = decode_rotated(np.ascontiguousarray(slots[:, :, kb:kb + kbv].transpose(1, 0, 2)),
                       np.ascontiguousarray(vn.T), cbV)
    return k, v


def _partial(q_rot, k, v, scale, mask=None):
    """attention_partial_reference (attention.py:190-236) in float64 for one
    (query rows, keys) block: (O_unnorm, m, l) with m in the natural domain."""
    s = (q_rot.astype(np.float64) @ k.astype(np.float64).T) * scale
    if mask is not None:
        s = np.where(mask, s, -np.inf)
    m = s.max(axis=-1) if s.shape[-1] else np.full(s.shape[0], -np.inf)
    with np.errstate(invalid="ignore"):
        p = np.exp(s - m[:, None])
    p = np.where(np.isnan(p), 0.0, p)
    return p @ v.astype(np.float64), m, p.sum(axis=-1)


def hybrid_prefill(q, cu_q, k_new, v_new, cache, block_table, seq_lens, cbK, cbV, R, *,
                   H_kv, block_size, scale=None):
    """Chunked prefill with a compressed prefix (cda_attn_v2.py:1023-1060):
    sequence b's queries (the last q_len of its seq_lens[b] positions) attend
    to keys [0, seq_lens[b] - q_len) decoded from the cache (all visible) and
    to the chunk's own K/V rotated to fp16(x R) (fa2_cda.py:256-287; causal),
    the two partials merged by merge_partials (attention.py:239-272), then
    out = fp16(fp16(O_rot) R^T).  q (T, H_q, 128), k_new/v_new (T, H_kv, 128)
    fp16; returns (T, H_q, 128) fp16."""
    q = np.asarray(q, dtype=np.float16)
    T, H_q, _ = q.shape
    gs = H_q // H_kv
    R32 = np.asarray(R, dtype=np.float32)
    if scale is None:
        scale = 1.0 / np.sqrt(D)
    q_rot = (q.astype(np.float32) @ R32).astype(np.float16)
    k_rot = (np.asarray(k_new, dtype=np.float16).astype(np.float32) @ R32).astype(np.float16)
    v_rot = (np.asarray(v_new, dtype=np.float16).astype(np.float32) @ R32).astype(np.float16)
    out = np.zeros((T, H_q, D), dtype=np.float16)
    for b in range(len(cu_q) - 1):
        q0, q1 = int(cu_q[b]), int(cu_q[b + 1])
        n = q1 - q0
        if n == 0:
            continue
        past = int(seq_lens[b]) - n
        kp, vp = paged_rows(cache, block_table, b, past, cbK, cbV, H_kv=H_kv,
                            block_size=block_size)
        causal = np.arange(n)[None, :] <= np.arange(n)[:, None]
        for hq in range(H_q):
            h = hq // gs
            qr = q_rot[q0:q1, hq]
            parts = [_partial(qr, kp[h], vp[h], scale),
                     _partial(qr, k_rot[q0:q1, h], v_rot[q0:q1, h], scale, causal)]
            o_rot = merge_partials(parts)
            out[q0:q1, hq] = (o_rot.astype(np.float32) @ R32.T).astype(np.float16)
    return out
