"""Closed-form and brute-force pins of the CPU checker (no reference needed).

Each check is chosen so that a plausible slip (a transposed operand, a
dropped term, a wrong tie rule, a wrong nibble order) fails it."""
from fractions import Fraction
import math

import numpy as np
import pytest

from oracle import cda_oracle as O
from oracle import synth

D = 128


def test_f64_to_f16_is_correctly_rounded():
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.standard_normal(200000) * 10.0 ** rng.integers(-9, 6, 200000),
        np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, 1e6, 2.0 ** -24, 2.0 ** -25,
                  2.0 ** -25 * 1.0000001, 3 * 2.0 ** -26, 1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11,
                  np.inf, -np.inf]),
    ])
    got = np.array([O.lib().cda_oracle_f64_to_f16(float(v)) for v in x], dtype=np.uint16)
    ref = x.astype(np.float16).view(np.uint16)      # numpy rounds to nearest-even
    assert np.array_equal(got, ref)


def test_hadamard_is_sylvester_and_orthonormal():
    H = O.hadamard128().astype(np.float64)
    h = H[0, 0]
    assert np.float32(h) == np.float32(1.0) / np.float32(math.sqrt(128))
    assert set(np.unique(np.abs(H))) == {h}
    assert np.array_equal(H, H.T)
    H2 = np.array([[1.0]])
    while H2.shape[0] < D:
        H2 = np.block([[H2, H2], [H2, -H2]])
    assert np.array_equal(np.sign(H), H2)
    np.testing.assert_allclose(H @ H.T, np.eye(D), atol=1e-6)


@pytest.mark.parametrize("L", [16, 4])
def test_quantize_is_nearest_with_lower_ties(codebooks, L):
    cb = codebooks["lloyd_beta16" if L == 16 else "lloyd_beta4"].astype(np.float32)
    rng = np.random.default_rng(L)
    x = rng.uniform(-1.0, 1.0, 200000).astype(np.float32)
    idx = O.quantize_unit(x, cb).astype(np.int64)
    d = np.abs(x.astype(np.float64)[:, None] - cb.astype(np.float64)[None, :])
    best = d.argmin(axis=1)                          # first minimum = lower index
    srt = np.sort(d, axis=1)
    clear = (srt[:, 1] - srt[:, 0]) > 1e-6
    assert np.array_equal(idx[clear], best[clear])
    # special cases: exact centroids, exact midpoints (-> lower), ends of range
    assert np.array_equal(O.quantize_unit(cb, cb), np.arange(L))
    mids = ((cb[:-1] + cb[1:]) * np.float32(0.5)).astype(np.float32)
    exact_mid = (mids - cb[:-1]) == (cb[1:] - mids)
    assert np.array_equal(O.quantize_unit(mids, cb)[exact_mid], np.arange(L - 1)[exact_mid])
    assert O.quantize_unit(np.float32([-1.0]), cb)[0] == 0
    assert O.quantize_unit(np.float32([1.0]), cb)[0] == L - 1


def test_pack_unpack_brute_force():
    allb = np.arange(256, dtype=np.uint8)[:, None]
    assert np.array_equal(O.pack_4bit(O.unpack_4bit(allb)), allb)
    assert np.array_equal(O.pack_2bit(O.unpack_2bit(allb)), allb)
    pairs = np.array([[a, b] for a in range(16) for b in range(16)], dtype=np.uint8)
    assert np.array_equal(O.pack_4bit(pairs)[:, 0], (pairs[:, 0] << 4) | pairs[:, 1])
    quads = np.array(np.meshgrid(*[range(4)] * 4, indexing="ij")).reshape(4, -1).T.astype(np.uint8)
    got = O.pack_2bit(quads)[:, 0]
    assert np.array_equal(got, (quads[:, 0] << 6) | (quads[:, 1] << 4) | (quads[:, 2] << 2) | quads[:, 3])


def _exact_row(x16):
    """Exact Fraction rotation of one fp16 row with the fp32 Hadamard entry."""
    h = Fraction(float(np.float32(O.hadamard128()[0, 0])))
    H = np.sign(O.hadamard128())
    xs = [Fraction(float(v)) for v in x16]
    return [h * sum(xs[i] * int(H[i, j]) for i in range(D)) for j in range(D)]


def _round_f16_exact(fr):
    """Round a Fraction to fp16 (nearest-even) by bracketing."""
    v = float(fr)
    cand = np.float16(v)
    best = None
    for c in (np.nextafter(cand, np.float16(-np.inf)), cand, np.nextafter(cand, np.float16(np.inf))):
        if not np.isfinite(c):
            continue
        err = abs(Fraction(float(c)) - fr)
        key = (err, int(np.float16(c).view(np.uint16)) & 1)
        if best is None or key < best[0]:
            best = (key, c)
    return best[1]


def test_encode_rotation_and_norm_within_fp32_error_bounds(codebooks):
    """x_rot is an fp32 recurrence of 128 fused multiply-adds rounded to fp16,
    the norm a 128-term fp32 sum of squares: each must lie within the textbook
    error bound of the exact value (rational arithmetic on random rows), so a
    dropped term, a wrong sign or a transposed operand fails."""
    x = synth.kv_with_outliers(11, (6, D))
    _, norm, xrot = O.encode(x, codebooks["lloyd_beta16"])
    u32 = Fraction(1, 2 ** 24)
    gamma = 128 * u32 / (1 - 128 * u32)
    for r in range(x.shape[0]):
        ex = _exact_row(x[r])
        h = Fraction(float(np.float32(1 / np.sqrt(128))))
        abs_sum = sum(abs(Fraction(float(v))) for v in x[r]) * h
        for j in range(D):
            got = Fraction(float(xrot[r, j]))
            ulp16 = Fraction(float(np.spacing(np.float16(abs(xrot[r, j])))))
            assert abs(got - ex[j]) <= gamma * abs_sum + ulp16 / 2 + Fraction(1, 2 ** 25)
        ss = sum(Fraction(float(v)) ** 2 for v in xrot[r])
        n = Fraction(float(norm[r]))
        # sum of squares: relative error <= gamma_129; sqrt and its rounding <= 2 u32
        lo, hi = ss * (1 - gamma * 2), ss * (1 + gamma * 2)
        assert lo * (1 - 4 * u32) <= n * n <= hi * (1 + 4 * u32)


def test_encode_decode_round_trip(codebooks):
    """Invariants: ||decode|| tracks norm * ||cb[idx]||, and the rotated-frame
    reconstruction is close to x_rot (cos >= 0.97 for the 16-level table)."""
    cb = codebooks["lloyd_beta16"]
    x = synth.normal_f16(12, (512, D))
    packed, norm, xrot = O.encode(x, cb)
    dec = O.decode_rotated(packed, norm, cb).astype(np.float64)
    xr = xrot.astype(np.float64)
    cos = (dec * xr).sum(-1) / np.linalg.norm(dec, axis=-1) / np.linalg.norm(xr, axis=-1)
    assert cos.min() > 0.97
    units = np.linalg.norm(cb[O.unpack_4bit(packed)].astype(np.float64), axis=-1)
    np.testing.assert_allclose(np.linalg.norm(dec, axis=-1), norm * units, rtol=2e-3)
    np.testing.assert_allclose(norm, np.linalg.norm(x.astype(np.float64), axis=-1), rtol=2e-3)


def _case(seed, seq_lens, H_kv=2, gs=4, bs=16):
    cb = np.load(__import__("pathlib").Path(__file__).parent / "golden" / "codebooks.npz")["lloyd_beta16"]
    B = len(seq_lens)
    N = max(seq_lens)
    k = synth.kv_with_outliers(seed, (B, H_kv, N, D))
    v = synth.normal_f16(seed + 1, (B, H_kv, N, D))
    q = synth.normal_f16(seed + 2, (B, H_kv * gs, D))
    kp, kn, _ = O.encode(k, cb)
    vp, vn, _ = O.encode(v, cb)
    W = (N + bs - 1) // bs + 1
    bt = synth.permuted_block_table(seed, B, W)
    cache = O.build_paged_cache(kp, kn, vp, vn, bt, bs, 16, num_blocks=B * W)
    return dict(cb=cb, q=q, kp=kp, kn=kn, vp=vp, vn=vn, bt=bt, cache=cache,
                sl=np.array(seq_lens, np.int32), H_kv=H_kv, gs=gs, bs=bs)


def test_decode_matches_fp64_textbook_attention():
    """Brute force: decode K/V (fp16), softmax(q K^T / sqrt(D)) V in float64,
    with the rotations and fp16 rounding points of attention_compressed."""
    c = _case(21, [37, 100])
    R = O.hadamard128().astype(np.float64)
    out = O.decode_paged(c["q"], c["cache"], c["bt"], c["sl"], c["cb"], c["cb"], O.hadamard128(),
                         H_kv=c["H_kv"], block_size=c["bs"]).astype(np.float64)
    for b, n in enumerate(c["sl"]):
        for hq in range(c["H_kv"] * c["gs"]):
            h = hq // c["gs"]
            K = O.decode_rotated(c["kp"][b, h, :n], c["kn"][b, h, :n], c["cb"]).astype(np.float64)
            V = O.decode_rotated(c["vp"][b, h, :n], c["vn"][b, h, :n], c["cb"]).astype(np.float64)
            qr = (c["q"][b, hq].astype(np.float64) @ R).astype(np.float32).astype(np.float16)
            s = K @ qr.astype(np.float64) / math.sqrt(D)
            p = np.exp(s - s.max())
            orot = ((p @ V) / p.sum()).astype(np.float32).astype(np.float16).astype(np.float64)
            ref = orot @ R.T
            np.testing.assert_allclose(out[b, hq], ref, atol=1e-3, rtol=0)


def test_k4v2_layout_decode_matches_fp64_textbook_attention(codebooks):
    """The legacy K4V2 slot (104 B: K 4-bit | V 2-bit | K norm | V norm,
    cda_attn_v2.py:29): the paged decode reads the fields at those offsets and
    decodes V with the 4-level codebook; checked by brute force as above."""
    cbk, cbv = codebooks["lloyd_beta16"], codebooks["lloyd_beta4"]
    B, H_kv, gs, bs, N = 2, 2, 4, 16, 90
    k = synth.kv_with_outliers(31, (B, H_kv, N, D))
    v = synth.normal_f16(32, (B, H_kv, N, D))
    q = synth.normal_f16(33, (B, H_kv * gs, D))
    kp, kn, _ = O.encode(k, cbk)
    vp, vn, _ = O.encode(v, cbv)
    W = (N + bs - 1) // bs
    bt = synth.permuted_block_table(34, B, W)
    cache = O.build_paged_cache(kp, kn, vp, vn, bt, bs, 16, num_blocks=B * W, Lv=4)
    assert cache.shape[-1] == 104
    sl = np.array([N, 41], np.int32)
    R = O.hadamard128().astype(np.float64)
    out = O.decode_paged(q, cache, bt, sl, cbk, cbv, O.hadamard128(), H_kv=H_kv,
                         block_size=bs).astype(np.float64)
    for b, n in enumerate(sl):
        for hq in range(H_kv * gs):
            h = hq // gs
            K = O.decode_rotated(kp[b, h, :n], kn[b, h, :n], cbk).astype(np.float64)
            V = O.decode_rotated(vp[b, h, :n], vn[b, h, :n], cbv).astype(np.float64)
            qr = (q[b, hq].astype(np.float64) @ R).astype(np.float32).astype(np.float16)
            s_ = K @ qr.astype(np.float64) / math.sqrt(D)
            p = np.exp(s_ - s_.max())
            orot = ((p @ V) / p.sum()).astype(np.float32).astype(np.float16).astype(np.float64)
            np.testing.assert_allclose(out[b, hq], orot @ R.T, atol=1e-3, rtol=0)


def test_split_merge_equals_single_pass():
    c = _case(22, [203])
    R = O.hadamard128()
    q_rot = (c["q"].astype(np.float64) @ R.astype(np.float64)).astype(np.float32).astype(np.float16)
    full = O.decode_paged(q_rot, c["cache"], c["bt"], c["sl"], c["cb"], c["cb"], R,
                          H_kv=c["H_kv"], block_size=c["bs"], rotated_io=True)
    for splits in (1, 2, 5, 13):
        chunk = -(-203 // splits)
        parts = [O.decode_partial(q_rot, c["cache"], c["bt"], c["sl"], c["cb"], c["cb"],
                                  H_kv=c["H_kv"], block_size=c["bs"], k0=s, k1=s + chunk)
                 for s in range(0, 203, chunk)]
        merged = O.merge_partials(parts)
        assert np.abs(merged.astype(np.float32) - full.astype(np.float32)).max() <= 1e-3
    # an empty window contributes nothing (m=-inf, l=0) and merges away
    empty = O.decode_partial(q_rot, c["cache"], c["bt"], c["sl"], c["cb"], c["cb"],
                             H_kv=c["H_kv"], block_size=c["bs"], k0=500, k1=600)
    assert np.all(np.isneginf(empty[1])) and np.all(empty[2] == 0)
    one = O.decode_partial(q_rot, c["cache"], c["bt"], c["sl"], c["cb"], c["cb"],
                           H_kv=c["H_kv"], block_size=c["bs"], k0=0, k1=203)
    assert np.array_equal(O.merge_partials([one, empty]), O.merge_partials([one]))


def test_rotated_frame_consistency():
    """attention in the unrotated frame == unrotate(attention in the rotated frame)."""
    c = _case(23, [150])
    R = O.hadamard128()
    q_rot = (c["q"].astype(np.float64) @ R.astype(np.float64)).astype(np.float32).astype(np.float16)
    a = O.decode_paged(c["q"], c["cache"], c["bt"], c["sl"], c["cb"], c["cb"], R,
                       H_kv=c["H_kv"], block_size=c["bs"])
    b = O.decode_paged(q_rot, c["cache"], c["bt"], c["sl"], c["cb"], c["cb"], R,
                       H_kv=c["H_kv"], block_size=c["bs"], rotated_io=True)
    ub = (b.astype(np.float64) @ R.astype(np.float64).T)
    np.testing.assert_allclose(a.astype(np.float64), ub, atol=2e-3)


def test_causal_prefill_last_row_is_decode():
    """The last query row of a causal prefill sees every key: it equals decode."""
    c = _case(24, [90])
    R = O.hadamard128()
    M = 7
    q = synth.normal_f16(99, (M, c["H_kv"] * c["gs"], D))
    pre = O.prefill_paged(q, np.array([0, M]), c["cache"], c["bt"], c["sl"], c["cb"], c["cb"], R,
                          H_kv=c["H_kv"], block_size=c["bs"])
    dec = O.decode_paged(q[M - 1:M], c["cache"], c["bt"], c["sl"], c["cb"], c["cb"], R,
                         H_kv=c["H_kv"], block_size=c["bs"])
    assert np.array_equal(pre[M - 1], dec[0])
    # row i sees keys [0, 90 - M + i]: equals decode with seq_len = 90 - M + i + 1
    for i in range(M):
        sl = np.array([90 - M + i + 1], np.int32)
        d = O.decode_paged(q[i:i + 1], c["cache"], c["bt"], sl, c["cb"], c["cb"], R,
                           H_kv=c["H_kv"], block_size=c["bs"])
        assert np.array_equal(pre[i], d[0])


def test_paged_rows_are_the_encoded_rows():
    """paged_rows reads sequence b's keys through the permuted block table:
    equal to decoding the encodings the cache was built from."""
    from tests.cases import make_hybrid_case
    c = make_hybrid_case(71, [3, 5], [37, 20], H_kv=2)
    kp, kn = c.k_enc
    for b, n in enumerate(c.seq_k):
        k, _ = O.paged_rows(c.cache, c.block_table, b, int(n), c.cb, c.cb, H_kv=2,
                            block_size=c.block_size)
        assert np.array_equal(k.view(np.uint16),
                              O.decode_rotated(kp[b, :, :n], kn[b, :, :n], c.cb).view(np.uint16))


def test_hybrid_merge_equals_one_softmax():
    """hybrid_prefill (two partials + merge_partials) equals one float64
    softmax over [decoded prefix; rotated raw chunk] with the prefix visible to
    every query and the chunk causal; and the no-prefix case reduces to plain
    causal attention over the raw chunk in the unrotated frame (R orthonormal:
    within fp16 rounding)."""
    from tests.cases import make_hybrid_case
    c = make_hybrid_case(72, [4, 6, 3], [30, 6, 19], H_kv=2, gs=4)
    R = O.hadamard128().astype(np.float64)
    s = 1.0 / np.sqrt(128)
    q_rot = (c.q.astype(np.float32) @ R.astype(np.float32)).astype(np.float16)
    k_rot = (c.k_new.astype(np.float32) @ R.astype(np.float32)).astype(np.float16)
    v_rot = (c.v_new.astype(np.float32) @ R.astype(np.float32)).astype(np.float16)
    for b in range(3):
        q0, q1 = c.cu_q[b], c.cu_q[b + 1]
        n = q1 - q0
        past = c.seq_k[b] - n
        kp, vp = O.paged_rows(c.cache, c.block_table, b, past, c.cb, c.cb, H_kv=2,
                              block_size=c.block_size)
        for hq in range(8):
            h = hq // 4
            K = np.concatenate([kp[h], k_rot[q0:q1, h]]).astype(np.float64)
            V = np.concatenate([vp[h], v_rot[q0:q1, h]]).astype(np.float64)
            sc = q_rot[q0:q1, hq].astype(np.float64) @ K.T * s
            vis = np.arange(past + n)[None, :] <= past + np.arange(n)[:, None]
            sc = np.where(vis, sc, -np.inf)
            p = np.exp(sc - sc.max(1, keepdims=True))
            o = ((p @ V) / p.sum(1, keepdims=True)).astype(np.float16)
            exp = (o.astype(np.float32) @ R.T.astype(np.float32)).astype(np.float16)
            got = c.expected[q0:q1, hq]
            assert np.abs(got.astype(np.float32) - exp.astype(np.float32)).max() <= 1e-3
            if past == 0:
                kk = c.k_new[q0:q1, h].astype(np.float64)
                vv = c.v_new[q0:q1, h].astype(np.float64)
                sc2 = np.where(vis, c.q[q0:q1, hq].astype(np.float64) @ kk.T * s, -np.inf)
                p2 = np.exp(sc2 - sc2.max(1, keepdims=True))
                o2 = (p2 @ vv) / p2.sum(1, keepdims=True)
                assert np.abs(got.astype(np.float64) - o2).max() <= 4e-3
