"""The torch-CPU restatement (oracle/torch_ref.py, the CPU baseline bench.py
times) against the reference-written fixtures: it must give the reference's
bits on this host's CPU."""
import json
from pathlib import Path

import numpy as np
import torch

from oracle import synth
from oracle import torch_ref as T

GOLD = Path(__file__).parent / "golden"


def test_hadamard_equals_reference(codebooks):
    assert np.array_equal(T.hadamard().numpy(), codebooks["hadamard128"])


def test_encode_rows_equal_reference(golden, codebooks):
    e = golden("encode.npz")
    cb = torch.from_numpy(codebooks["lloyd_beta16"])
    codes, norm = T.encode(torch.from_numpy(e["x"]), cb, T.hadamard())
    assert np.array_equal(codes.numpy(), e["k4_idx"])
    assert np.array_equal(norm.numpy().view(np.uint32), e["k4_norm"].view(np.uint32))
    dec = T.decode_rows(torch.from_numpy(e["k4_idx"]), torch.from_numpy(e["k4_norm"]), cb)
    assert np.array_equal(dec.numpy().view(np.uint16), e["k4_dec_rot"].view(np.uint16))


def test_config0_equals_reference(golden, codebooks):
    g = golden("attn_cfg0.npz")
    meta = json.loads((GOLD / "attn_cfg0.json").read_text())
    seed, N = meta["seed"], meta["N"]
    cb = torch.from_numpy(codebooks["lloyd_beta16"])
    H = T.hadamard()
    k = torch.from_numpy(synth.kv_with_outliers(seed, (1, 8, N, 128)))
    v = torch.from_numpy(synth.normal_f16(seed + 1, (1, 8, N, 128)))
    kc, kn = T.encode(k, cb, H)
    vc, vn = T.encode(v, cb, H)
    assert np.array_equal(kc.numpy(), g["k_idx"]) and np.array_equal(vc.numpy(), g["v_idx"])
    assert np.array_equal(kn.numpy(), g["k_norm"]) and np.array_equal(vn.numpy(), g["v_norm"])
    out = T.attention_compressed(torch.from_numpy(g["q"]), kc, kn, vc, vn, cb, H, 4)
    assert np.array_equal(out.numpy().view(np.uint16), g["out"].view(np.uint16))


def _uniform16():
    return ((torch.arange(16, dtype=torch.float64) * 2 + 1) / 16 - 1).float()


def test_qk_scores_uniform4_closed_form():
    """Score-domain QK (attention.py:101-152) equals q_rot . (cb[code] * norm)
    * scale for the uniform codebook cb[i] = (2i + 1)/16 - 1, computed in
    float64 from the codes; the causal mask over a key window is checked
    entry by entry (key_start + k visible to query m iff <= m + q_offset)."""
    g = torch.Generator().manual_seed(5)
    B, H_kv, gs, M_q, M_k = 2, 2, 4, 5, 37
    q = torch.randn(B, H_kv * gs, M_q, 128, generator=g).half()
    idx = torch.randint(0, 256, (B, H_kv, M_k, 64), generator=g, dtype=torch.uint8)
    norm = torch.rand(B, H_kv, M_k, generator=g) * 20 + 0.1
    cb = _uniform16()
    sc = T.qk_scores_uniform4(q, idx, norm, gs)
    k = cb.double()[T.unpack4(idx).long()] * norm.double().unsqueeze(-1)
    exp = torch.einsum("bhgmd,bhkd->bhgmk", q.double().view(B, H_kv, gs, M_q, 128), k) / 128 ** 0.5
    assert torch.allclose(sc.double(), exp, rtol=1e-5, atol=1e-4)
    ks, ke, qo = 7, 30, 12
    sc2 = T.qk_scores_uniform4(q, idx, norm, gs, causal=True, q_offset=qo, key_start=ks,
                               key_end=ke)
    for m in range(M_q):
        for kk in range(ke - ks):
            masked = bool(torch.isinf(sc2[..., m, kk]).all())
            assert masked == (ks + kk > m + qo)
            if not masked:
                assert torch.equal(sc2[..., m, kk], sc[..., m, ks + kk])


def test_attention_qk_uniform4_matches_decoded_k():
    """With score-domain QK the attention differs from the decoded-K path
    (attention.py:306-346) only by the fp16 rounding of K: within 2e-3."""
    g = torch.Generator().manual_seed(6)
    B, H_kv, gs, M_k = 1, 2, 4, 300
    cb = _uniform16()
    k = torch.randn(B, H_kv, M_k, 128, generator=g).half()
    v = torch.randn(B, H_kv, M_k, 128, generator=g).half()
    H = T.hadamard()
    kc, kn = T.encode(k, cb, H)
    vc, vn = T.encode(v, cb, H)
    q_rot = T.rotate(torch.randn(B, H_kv * gs, 1, 128, generator=g).half(), H)
    got = T.attention_qk_uniform4(q_rot, kc, kn, vc, vn, cb, gs)
    ref = T.gqa_attention(q_rot, T.decode_rows(kc, kn, cb), T.decode_rows(vc, vn, cb), gs)
    assert (got.float() - ref.float()).abs().max() <= 2e-3
