"""The decoded K/V rows round twice, as the reference does: the fp32 product
cb[code] * norm, then .to(torch.float16) (compression.py:355-359).  The norms
here are picked so that rounding the exact product once to fp16 gives a
different value for some code: a kernel whose multiply and conversion fuse
into one rounding (v_fma_mixlo_f16) fails these rows, random data almost
never shows it (about 1 row in 1200)."""
import numpy as np
import pytest
import torch

from oracle import cda_oracle as O
from tests.cases import synth_cb


def _tricky_rows(cb, n_rows=64, seed=11):
    """(codes (n_rows, 128), norms (n_rows,)) with every row holding a code
    whose single- and double-rounded fp16 values differ."""
    rng = np.random.default_rng(seed)
    norms = []
    while len(norms) < n_rows:
        n = (rng.random(20000) * 60 + 0.5).astype(np.float32)
        prod = cb[None, :].astype(np.float64) * n[:, None].astype(np.float64)   # exact
        bad = (prod.astype(np.float16) != prod.astype(np.float32).astype(np.float16)).any(axis=1)
        norms.extend(n[bad].tolist())
    norms = np.asarray(norms[:n_rows], dtype=np.float32)
    codes = np.stack([rng.permutation(np.arange(128) % cb.size) for _ in range(n_rows)])
    return codes.astype(np.uint8), norms


def _expected(cb, codes, norms):
    return (cb[codes] * norms[:, None]).astype(np.float16)          # fp32 product, then fp16


def test_tricky_rows_need_two_roundings():
    """CPU pin of the data and the checker: one rounding differs on every
    row, the checker's decode rounds twice."""
    cb = synth_cb().astype(np.float32)
    codes, norms = _tricky_rows(cb)
    once = (cb[codes].astype(np.float64) * norms[:, None].astype(np.float64)).astype(np.float16)
    twice = _expected(cb, codes, norms)
    assert (once != twice).any(axis=1).all()
    packed = O.pack_4bit(codes)
    dec = O.decode_rotated(packed[:, None], norms[:, None], cb)[:, 0]
    assert np.array_equal(dec.view(np.uint16), twice.view(np.uint16))


@pytest.mark.gpu
def test_dequantize_rows_rounds_twice(gpu):
    from sub0_amd import _native
    print("[double-rounding] dequantize_rows", flush=True)
    cb = synth_cb().astype(np.float32)
    codes, norms = _tricky_rows(cb)
    packed = O.pack_4bit(codes)
    out = _native.dequantize_rows(torch.from_numpy(packed[:, None].copy()).to(gpu),
                                  torch.from_numpy(norms[:, None].copy()).to(gpu),
                                  torch.from_numpy(cb).to(gpu))
    got = out[:, 0].cpu().numpy()
    assert np.array_equal(got.view(np.uint16), _expected(cb, codes, norms).view(np.uint16))


@pytest.mark.gpu
def test_dense_loader_rounds_twice(gpu):
    """paged_cache_to_dense_rotated (the prefill's dense bridge) on a paged
    cache of these rows, K and V."""
    from sub0_amd import _native
    print("[double-rounding] paged_to_dense", flush=True)
    cb = synth_cb().astype(np.float32)
    n = 64
    kc, kn = _tricky_rows(cb, n, seed=12)
    vc, vn = _tricky_rows(cb, n, seed=13)
    H = 8                                                       # the same rows for every head
    kp = np.broadcast_to(O.pack_4bit(kc)[None, None], (1, H, n, 64)).copy()
    vp = np.broadcast_to(O.pack_4bit(vc)[None, None], (1, H, n, 64)).copy()
    knh = np.broadcast_to(kn[None, None], (1, H, n)).copy()
    vnh = np.broadcast_to(vn[None, None], (1, H, n)).copy()
    bt = np.arange(n // 16, dtype=np.int32)[None][:, ::-1].copy()   # pages in reverse order
    cache = O.build_paged_cache(kp, knh, vp, vnh, bt, 16, 16)
    dev = gpu
    k_rot, v_rot = _native.paged_to_dense(torch.from_numpy(cache).to(dev), torch.from_numpy(bt).to(dev),
                                          torch.tensor([n], dtype=torch.int32, device=dev),
                                          torch.from_numpy(cb).to(dev), torch.from_numpy(cb).to(dev),
                                          block_size=16, max_seq_len=n)
    for got, codes, norms in ((k_rot, kc, kn), (v_rot, vc, vn)):
        got = got.cpu().numpy().reshape(n, H, 128)
        exp = _expected(cb, codes, norms)
        for h in range(H):
            assert np.array_equal(got[:, h].view(np.uint16), exp.view(np.uint16)), f"head {h}"
