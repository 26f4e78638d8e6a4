"""GPU parity of the hybrid chunked prefill (compressed prefix + the chunk's
raw K/V, log-sum-exp merge; cda_attn_v2.py:1023-1060) against the CPU
checker's ``hybrid_prefill``, through the C ABI, the reference-shaped
``hybrid_attn_v1`` and the backend's raw-K/V routes.

Tolerance: 2e-3 max-abs on fp16 outputs; the checker
computes in float64 from the same cache and the same raw K/V."""
import numpy as np
import pytest
import torch

from tests.cases import make_hybrid_case, raw_causal_attention

pytestmark = pytest.mark.gpu
TOL = 2e-3


def _dev(x, dev):
    return torch.from_numpy(np.ascontiguousarray(x)).to(dev)


def _check(out, exp):
    assert np.isfinite(out).all(), "non-finite output"
    err = float(np.abs(out.astype(np.float32) - exp.astype(np.float32)).max()) if out.size else 0.0
    assert err <= TOL, f"max abs err {err}"


CASES = [
    # name, seq_q, seq_k, H_kv, gs
    ("one_seq", [40], [300], 8, 4),
    ("ragged", [17, 64, 1, 129], [100, 64, 50, 300], 8, 4),   # second: no prefix
    ("long_prefix_split", [16, 3], [5000, 2100], 8, 4),        # prefix keys split
    ("big_chunk", [600], [700], 8, 4),
    ("gs8", [70, 33], [150, 33], 4, 8),
    ("hkv2", [129], [1000], 2, 4),
    # >= 256 workgroups on both sides: no key split, the prefix kernel merges
    # the chunk's partial in its epilogue (no combine launch)
    ("no_split_merge", [1024, 1040], [2048, 1500], 8, 4),
]


@pytest.mark.parametrize("name,seq_q,seq_k,H_kv,gs", CASES, ids=[c[0] for c in CASES])
def test_hybrid_matches_checker(gpu, name, seq_q, seq_k, H_kv, gs):
    from sub0_amd import _native
    print(f"[hybrid] case={name} seq_q={seq_q} seq_k={seq_k}", flush=True)
    c = make_hybrid_case(5000 + len(name), seq_q, seq_k, H_kv=H_kv, gs=gs)
    q = _dev(c.q, gpu)
    out = torch.full_like(q, float("nan"))
    cb = _dev(c.cb, gpu)
    _native.prefill_hybrid(q, _dev(c.k_new, gpu), _dev(c.v_new, gpu), _dev(c.cache, gpu),
                           _dev(c.block_table, gpu), _dev(c.cu_q, gpu), _dev(c.seq_k, gpu), cb, cb,
                           out, block_size=c.block_size, max_query_len=int(max(seq_q)),
                           max_seq_len=int(max(seq_k)), scale=1.0 / np.sqrt(128))
    torch.cuda.synchronize()
    _check(out.cpu().numpy(), c.expected)


def test_hybrid_wrapper_and_small_bound(gpu):
    """hybrid_attn_v1 with the reference's keyword call, a 4-D cache view and
    a max_seq_len bound below the longest sequence (costs speed, not keys)."""
    from sub0_amd.cda.kernels_cuda.wrappers import hybrid_attn_v1
    seq_q, seq_k = [20, 5], [900, 40]
    print(f"[hybrid] wrapper seq_q={seq_q} seq_k={seq_k}", flush=True)
    c = make_hybrid_case(5100, seq_q, seq_k)
    q = _dev(c.q, gpu)
    cache = _dev(c.cache, gpu)
    cache4 = cache.view(-1, c.block_size, *cache.shape[1:])
    cb = _dev(c.cb, gpu)
    for bound in (None, 100):
        out = torch.full_like(q, float("nan"))
        hybrid_attn_v1(q, _dev(c.k_new, gpu), _dev(c.v_new, gpu), out, cache4,
                       _dev(c.block_table, gpu), cu_seqlens_q=_dev(c.cu_q, gpu),
                       seq_lens=_dev(c.seq_k, gpu), cb_K=cb, cb_V=cb, rotation_fp32=None,
                       rotation_fp16=None, scale=1.0 / np.sqrt(128), group_size=4,
                       block_size=c.block_size, max_seq_len=bound,
                       max_query_len=None if bound is None else 20)
        torch.cuda.synchronize()
        _check(out.cpu().numpy(), c.expected)


def test_rawkv_no_past_routes(gpu):
    """No prefix: fa2_raw_prefill_varlen_v1 (no rotation) against plain
    float64 causal attention of the raw inputs; fa2_cda_prefill_rawkv_varlen_v1
    (rotated raw K/V, the fused kernel) against the checker's rotated-frame
    hybrid_prefill with an empty prefix."""
    from sub0_amd.cda.algorithm.compression import hadamard_matrix
    from sub0_amd.cda.kernels_cuda.fa2_cda import (fa2_cda_prefill_rawkv_varlen_v1,
                                                   fa2_raw_prefill_varlen_v1)
    seq = [33, 200, 1]
    print(f"[hybrid] rawkv no-past seq={seq}", flush=True)
    c = make_hybrid_case(5200, seq, seq)
    q = _dev(c.q, gpu)
    k, v = _dev(c.k_new, gpu), _dev(c.v_new, gpu)
    cu = _dev(c.cu_q, gpu)
    sl = _dev(c.seq_k, gpu)
    out = torch.full_like(q, float("nan"))
    fa2_raw_prefill_varlen_v1(q, k, v, cu, out, group_size=4, max_query_len=200)
    torch.cuda.synchronize()
    _check(out.cpu().numpy(), raw_causal_attention(c.q, c.cu_q, c.k_new, c.v_new))
    out2 = torch.full_like(q, float("nan"))
    fa2_cda_prefill_rawkv_varlen_v1(q, k, v, cu, sl, out2,
                                    rotation_fp32=hadamard_matrix(128).to(gpu), group_size=4,
                                    max_query_len=200, max_seq_len=200)
    torch.cuda.synchronize()
    _check(out2.cpu().numpy(), c.expected)
