"""The CPU checker against the reference's own outputs (golden fixtures written
by tests/golden/make_golden.py from cda/algorithm) -- pins the oracle."""
import json
from pathlib import Path

import numpy as np
import pytest

from oracle import cda_oracle as O
from oracle import synth

GOLD = Path(__file__).parent / "golden"


def test_hadamard_matches_reference(codebooks):
    assert np.array_equal(O.hadamard128(), codebooks["hadamard128"])


@pytest.mark.parametrize("L", [16, 4])
def test_uniform_centroids_match_reference(codebooks, L):
    assert np.array_equal(O.uniform_centroids(L), codebooks[f"uniform{L}"])


@pytest.mark.parametrize("name,cbkey", [("cb16", "lloyd_beta16"), ("cb4", "lloyd_beta4")])
def test_quantize_matches_reference(golden, codebooks, name, cbkey):
    """Centroids, exact midpoints (ties -> lower), their fp32 neighbours, +-1, +-0."""
    q = golden("quantize.npz")
    got = O.quantize_unit(q[f"{name}_x"], codebooks[cbkey])
    assert np.array_equal(got, q[f"{name}_idx"])


@pytest.mark.parametrize("tag,cbkey", [("k4", "lloyd_beta16"), ("k2", "lloyd_beta4")])
def test_encode_indices_match_reference(golden, codebooks, tag, cbkey):
    """Packed indices are bit-exact on all 1032 fixture rows (1024 outlier rows
    + 8 edge rows: zero, constant, subnormal, fp16 overflow, one-hot, ramp)."""
    e = golden("encode.npz")
    packed, norm, xrot = O.encode(e["x"], codebooks[cbkey])
    assert np.array_equal(packed, e[f"{tag}_idx"])
    assert np.array_equal(norm.view(np.uint32), e[f"{tag}_norm"].view(np.uint32))
    # The 0 row clamps to 1e-12 and the overflow row gives inf in both.
    assert norm[1024] == np.float32(1e-12)
    assert np.isinf(norm[1027])


def test_rotation_matches_reference_bit_for_bit(golden):
    """x_rot: the fp32 fma chain in k order reproduces the reference's batched
    MKL sgemm rounding on every element (fp16 bit patterns, incl. the fp16
    overflow of the +-60000 edge row)."""
    e = golden("encode.npz")
    _, _, xrot = O.encode(e["x"], np.linspace(-1, 1, 16).astype(np.float32))
    assert np.array_equal(xrot.view(np.uint16), e["x_rot"].view(np.uint16))


def test_attention_fixture_encodings_match_reference(golden, codebooks):
    """The K and V encodings stored in the attention fixtures (GQA 4, GQA 8,
    causal): indices and fp32 norms bit for bit."""
    cb = codebooks["lloyd_beta16"]
    cases = (("attn_gs4.npz", 2001), ("attn_gs8.npz", 2002), ("attn_causal.npz", 2003))
    for fname, seed in cases:
        a = golden(fname)
        B, H_q, H_kv, N = (int(v) for v in a["meta"][:4])
        k = synth.kv_with_outliers(seed, (B, H_kv, N, 128))
        v = synth.normal_f16(seed + 1, (B, H_kv, N, 128))
        for x, tag in ((k, "k"), (v, "v")):
            p, n, _ = O.encode(x, cb)
            assert np.array_equal(p, a[f"{tag}_idx"]), (fname, tag)
            assert np.array_equal(n.view(np.uint32), a[f"{tag}_norm"].view(np.uint32)), (fname, tag)


@pytest.mark.parametrize("tag,cbkey", [("k4", "lloyd_beta16"), ("k2", "lloyd_beta4")])
def test_decode_rotated_matches_reference(golden, codebooks, tag, cbkey):
    e = golden("encode.npz")
    d = O.decode_rotated(e[f"{tag}_idx"], e[f"{tag}_norm"], codebooks[cbkey])
    assert np.array_equal(d.view(np.uint16), e[f"{tag}_dec_rot"].view(np.uint16))


def test_uniform_codebook_encode_matches_reference(golden, codebooks):
    e = golden("encode.npz")
    packed, _, _ = O.encode(e["x"][:256], codebooks["uniform16"])
    assert np.array_equal(packed, e["uniform_k4_idx"])


def _paged(a, seed, bs=16, L=16):
    B, H_q, H_kv, N = (int(v) for v in a["meta"][:4])
    nb = (N + bs - 1) // bs
    bt = synth.permuted_block_table(seed, B, nb)
    cache = O.build_paged_cache(a["k_idx"], a["k_norm"], a["v_idx"], a["v_norm"], bt, bs, L)
    return B, H_q, H_kv, N, bt, cache


@pytest.mark.parametrize("fname,tol", [("attn_gs4.npz", 1e-4), ("attn_gs8.npz", 5e-4)])
def test_attention_matches_reference(golden, codebooks, fname, tol):
    a = golden(fname)
    cb, R = codebooks["lloyd_beta16"], codebooks["hadamard128"]
    B, H_q, H_kv, N, bt, cache = _paged(a, 7)
    sl = np.full(B, N, np.int32)
    out = O.decode_paged(a["q"][:, :, 0], cache, bt, sl, cb, cb, R, H_kv=H_kv, block_size=16)
    assert np.abs(out.astype(np.float32) - a["out"][:, :, 0].astype(np.float32)).max() <= tol
    outr = O.decode_paged(a["q_rot"][:, :, 0], cache, bt, sl, cb, cb, R, H_kv=H_kv,
                          block_size=16, rotated_io=True)
    assert np.abs(outr.astype(np.float32) - a["out_rot"][:, :, 0].astype(np.float32)).max() <= tol


@pytest.mark.parametrize("fname", ["attn_gs4.npz", "attn_gs8.npz"])
def test_split_k_partials_and_merge_match_reference(golden, codebooks, fname):
    a = golden(fname)
    cb = codebooks["lloyd_beta16"]
    B, H_q, H_kv, N, bt, cache = _paged(a, 7)
    sl = np.full(B, N, np.int32)
    k_splits, k0, k1 = (int(v) for v in a["meta"][7:10])
    o, m, l = O.decode_partial(a["q_rot"][:, :, 0], cache, bt, sl, cb, cb, H_kv=H_kv,
                               block_size=16, k0=k0, k1=k1)
    np.testing.assert_allclose(o, a["part_o"][:, :, 0], rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(m, a["part_m"][:, :, 0], rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(l, a["part_l"][:, :, 0], rtol=1e-5)
    chunk = (N + k_splits - 1) // k_splits
    parts = [O.decode_partial(a["q_rot"][:, :, 0], cache, bt, sl, cb, cb, H_kv=H_kv,
                              block_size=16, k0=s, k1=min(s + chunk, N))
             for s in range(0, N, chunk)]
    merged = O.merge_partials(parts)
    assert np.abs(merged.astype(np.float32) - a["split_out"][:, :, 0].astype(np.float32)).max() <= 5e-4


def test_causal_prefill_matches_reference(golden, codebooks):
    a = golden("attn_causal.npz")
    cb, R = codebooks["lloyd_beta16"], codebooks["hadamard128"]
    B, H_q, H_kv, N, bt, cache = _paged(a, 9)
    M = int(a["meta"][4])
    q = a["q"][0].transpose(1, 0, 2).copy()           # (M, H_q, D)
    out = O.prefill_paged(q, np.array([0, M]), cache, bt, np.array([N]), cb, cb, R,
                          H_kv=H_kv, block_size=16)
    ref = a["out"][0].transpose(1, 0, 2).astype(np.float32)
    assert np.abs(out.astype(np.float32) - ref).max() <= 1e-3


def test_config0_encode_and_attention(golden, codebooks):
    """BASELINE config 0 (B=1, 32/8 heads, N=4096, outliers): the checker's
    encode equals the reference's (65536 rows per role: every index byte and
    every fp32 norm bit), and the attention over the reference's own cache
    matches its output."""
    g = golden("attn_cfg0.npz")
    meta = json.loads((GOLD / "attn_cfg0.json").read_text())
    B, H_kv, N, seed = meta["B"], meta["H_kv"], meta["N"], meta["seed"]
    cb, R = codebooks["lloyd_beta16"], codebooks["hadamard128"]
    k = synth.kv_with_outliers(seed, (B, H_kv, N, 128))
    v = synth.normal_f16(seed + 1, (B, H_kv, N, 128))
    q = synth.normal_f16(seed + 2, (B, 32, 1, 128))
    assert np.array_equal(q, g["q"])
    for x, ref_idx, ref_norm in ((k, g["k_idx"], g["k_norm"]), (v, g["v_idx"], g["v_norm"])):
        packed, norm, _ = O.encode(x, cb)
        assert np.array_equal(packed, ref_idx)
        assert np.array_equal(norm.view(np.uint32), ref_norm.view(np.uint32))
    bt = synth.permuted_block_table(seed, B, N // 16)
    cache = O.build_paged_cache(g["k_idx"], g["k_norm"], g["v_idx"], g["v_norm"], bt, 16, 16)
    out = O.decode_paged(g["q"][:, :, 0], cache, bt, np.full(B, N, np.int32), cb, cb, R,
                         H_kv=H_kv, block_size=16)
    assert np.abs(out.astype(np.float32) - g["out"][:, :, 0].astype(np.float32)).max() <= 2e-4
