"""GPU parity of the score-domain QK (attention.py:101-187) for the 16-level
uniform K codebook: the contiguous-layout scores kernel and attention
against the torch-CPU restatement (oracle/torch_ref.py, pinned by closed
forms in tests/test_torch_ref.py), and the paged decode option
(decode_hmma_v1(..., qk_without_k_decode=True)) against the same
restatement run per sequence.

Tolerances: scores rtol 1e-4 / atol 1e-3 (fp32 accumulation order); attention
outputs 2e-3 max-abs on fp16."""
import numpy as np
import pytest
import torch

from oracle import cda_oracle as O
from oracle import synth
from oracle import torch_ref as T

pytestmark = pytest.mark.gpu
TOL = 2e-3


def _uniform16():
    return torch.from_numpy(O.uniform_centroids(16).astype(np.float32))


def _slots(seed, B, H_kv, M_k):
    g = torch.Generator().manual_seed(seed)
    cb = _uniform16()
    H = T.hadamard()
    k = torch.from_numpy(synth.kv_with_outliers(seed, (B, H_kv, M_k, 128)))
    v = torch.randn(B, H_kv, M_k, 128, generator=g).half()
    kc, kn = T.encode(k, cb, H)
    vc, vn = T.encode(v, cb, H)
    return kc, kn, vc, vn, cb, g


@pytest.mark.parametrize("causal,window", [(False, None), (True, (40, 290, 260))],
                         ids=["full", "causal_window"])
def test_scores_kernel_matches_restatement(gpu, causal, window):
    from sub0_amd.cda.algorithm.attention import qk_scores_uniform_4bit_without_k_decode
    from sub0_amd.cda.algorithm.compression import CompressedSlot
    print(f"[score] scores kernel causal={causal} window={window}", flush=True)
    B, H_kv, gs, M_q, M_k = 2, 2, 4, 7, 300
    kc, kn, _, _, _, g = _slots(11, B, H_kv, M_k)
    q_rot = T.rotate(torch.randn(B, H_kv * gs, M_q, 128, generator=g).half(), T.hadamard())
    kw = {}
    if window:
        kw = dict(key_start=window[0], key_end=window[1], q_offset=window[2])
    exp = T.qk_scores_uniform4(q_rot, kc, kn, gs, causal=causal, **kw)
    exp = exp.reshape(B, H_kv * gs, M_q, -1)
    got = qk_scores_uniform_4bit_without_k_decode(
        q_rot.to(gpu), CompressedSlot(kc.to(gpu), kn.to(gpu)), group_size=gs, causal=causal,
        **kw).cpu()
    assert torch.equal(torch.isinf(got), torch.isinf(exp))
    fin = ~torch.isinf(exp)
    assert torch.allclose(got[fin], exp[fin], rtol=1e-4, atol=1e-3)


def test_scores_attention_matches_restatement(gpu):
    from sub0_amd.cda.algorithm.attention import (
        attention_compressed_rotated_reference_qk_without_k_decode)
    from sub0_amd.cda.algorithm.compression import CompressedSlot
    print("[score] attention", flush=True)
    B, H_kv, gs, M_q, M_k = 1, 2, 8, 3, 513
    kc, kn, vc, vn, cb, g = _slots(12, B, H_kv, M_k)
    q_rot = T.rotate(torch.randn(B, H_kv * gs, M_q, 128, generator=g).half(), T.hadamard())
    exp = T.attention_qk_uniform4(q_rot, kc, kn, vc, vn, cb, gs, causal=True, q_offset=510)
    got = attention_compressed_rotated_reference_qk_without_k_decode(
        q_rot.to(gpu), CompressedSlot(kc.to(gpu), kn.to(gpu)), CompressedSlot(vc.to(gpu), vn.to(gpu)),
        cb_V=cb.to(gpu), group_size=gs, causal=True, q_offset=510).cpu()
    assert (got.float() - exp.float()).abs().max() <= TOL


def _paged_case(seed, seq_lens, gs, cb_v_np, block_size=16):
    """Uniform-K paged cache (8 KV heads), queries and the expected decode:
    the restatement's score-domain attention per sequence, unrotated."""
    seq_lens = np.asarray(seq_lens, np.int32)
    B, H_kv = len(seq_lens), 8
    nmax = int(seq_lens.max())
    W = (nmax + block_size - 1) // block_size + 2
    bt = synth.permuted_block_table(seed, B, W)
    cbk = O.uniform_centroids(16).astype(np.float32)
    k = synth.kv_with_outliers(seed, (B, H_kv, nmax, 128))
    v = synth.normal_f16(seed + 1, (B, H_kv, nmax, 128))
    q = synth.normal_f16(seed + 2, (B, H_kv * gs, 128))
    kp, kn, _ = O.encode(k, cbk)
    vp, vn, _ = O.encode(v, cb_v_np)
    cache = O.build_paged_cache(kp, kn, vp, vn, bt, block_size, 16, num_blocks=B * W)
    H = T.hadamard()
    exp = np.zeros(q.shape, np.float16)
    for b, n in enumerate(seq_lens):
        q_rot = T.rotate(torch.from_numpy(q[b:b + 1, :, None]), H)
        o = T.attention_qk_uniform4(q_rot, torch.from_numpy(kp[b:b + 1, :, :n]),
                                    torch.from_numpy(kn[b:b + 1, :, :n]),
                                    torch.from_numpy(vp[b:b + 1, :, :n]),
                                    torch.from_numpy(vn[b:b + 1, :, :n]),
                                    torch.from_numpy(cb_v_np), gs)
        exp[b] = T.unrotate(o, H)[0, :, 0].numpy()
    return q, cache, bt, seq_lens, cbk, exp


@pytest.mark.parametrize("gs", [4, 8])
@pytest.mark.parametrize("v_cb", ["uniform", "lloyd"])
def test_decode_uniform_qk_matches_restatement(gpu, codebooks, gs, v_cb):
    from sub0_amd.cda.kernels_cuda.wrappers import decode_hmma_v1
    from sub0_amd.cda.algorithm.compression import hadamard_matrix
    seq = [1, 77, 1000, 4100]
    print(f"[score] decode gs={gs} V codebook={v_cb} seq={seq}", flush=True)
    cbv = (O.uniform_centroids(16) if v_cb == "uniform" else codebooks["lloyd_beta16"]).astype(np.float32)
    q, cache, bt, sl, cbk, exp = _paged_case(900 + gs, seq, gs, cbv)
    d = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(gpu)
    out = torch.full(q.shape, float("nan"), dtype=torch.float16, device=gpu)
    R = hadamard_matrix(128).to(gpu)
    decode_hmma_v1(d(q), d(cache), d(bt), d(sl), out, cb_K=d(cbk), cb_V=d(cbv),
                   rotation_fp32=R, rotation_fp16=R.half(), group_size=gs, block_size=16,
                   max_seq_len=int(sl.max()), qk_without_k_decode=True)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    assert np.isfinite(got).all()
    err = float(np.abs(got.astype(np.float32) - exp.astype(np.float32)).max())
    assert err <= TOL, f"max abs err {err}"


def test_decode_uniform_qk_rejects_other_codebooks_and_shapes(gpu, codebooks):
    """A non-uniform cb_K gives NaN (checked on the device); H_kv != 8 is an
    error from the C ABI."""
    from sub0_amd import _native
    lloyd = codebooks["lloyd_beta16"].astype(np.float32)
    q, cache, bt, sl, cbk, _ = _paged_case(950, [50, 200], 4, lloyd)
    d = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(gpu)
    R = torch.from_numpy(O.hadamard128().astype(np.float32)).to(gpu)
    out = torch.zeros(q.shape, dtype=torch.float16, device=gpu)
    _native.decode(d(q), d(cache), d(bt), d(sl), d(lloyd), d(lloyd), R, None, out, group_size=4,
                   block_size=16, tile_n=0, max_seq_len=200, scale=1 / np.sqrt(128),
                   uniform_qk=True)
    torch.cuda.synchronize()
    assert torch.isnan(out).all()
    with pytest.raises(ValueError, match="page-streaming"):
        _native.decode(d(q[:, :8]), d(cache[:, :2]), d(bt), d(sl), d(cbk), d(cbk), R, None,
                       out[:, :8].contiguous(), group_size=4, block_size=16, tile_n=0,
                       max_seq_len=200, scale=1 / np.sqrt(128), uniform_qk=True)
