"""GPU fused paged encode: bit-exact against the CPU checker (through the C ABI)."""
import numpy as np
import pytest
import torch

from oracle import cda_oracle as O
from oracle import synth

pytestmark = pytest.mark.gpu


def expected_cache(k, v, slots, cb, num_slots, slot_bytes, sentinel, cb_v=None):
    T, H_kv, _ = k.shape
    kp, kn, _ = O.encode(k, cb)
    vp, vn, _ = O.encode(v, cb if cb_v is None else cb_v)
    kb = kp.shape[-1]
    cache = np.full((num_slots, H_kv, slot_bytes), sentinel, dtype=np.uint8)
    for t in range(T):
        s = slots[t]
        if s < 0:
            continue
        cache[s, :, :kb] = kp[t]
        cache[s, :, kb:2 * kb] = vp[t]
        cache[s, :, 2 * kb:2 * kb + 4] = kn[t].astype(np.float32).view(np.uint8).reshape(H_kv, 4)
        cache[s, :, 2 * kb + 4:2 * kb + 8] = vn[t].astype(np.float32).view(np.uint8).reshape(H_kv, 4)
    return cache


def run_gpu_encode(dev, k, v, slots, cb, num_slots, slot_bytes, sentinel, cb_v=None):
    from sub0_amd import _native
    cache = torch.full((num_slots, k.shape[1], slot_bytes), sentinel, dtype=torch.uint8,
                       device=dev)
    cbt = torch.from_numpy(cb).to(dev)
    cbv = cbt if cb_v is None else torch.from_numpy(cb_v).to(dev)
    _native.paged_encode(torch.from_numpy(k).to(dev), torch.from_numpy(v).to(dev),
                         torch.from_numpy(slots.astype(np.int32)).to(dev), cache, cbt, cbv)
    torch.cuda.synchronize()
    return cache.cpu().numpy()


@pytest.mark.parametrize("levels,slot_bytes", [(16, 144), (4, 80), (16, 160)])
def test_encode_bit_exact(gpu, codebooks, levels, slot_bytes):
    print(f"[encode] levels={levels} slot_bytes={slot_bytes}", flush=True)
    cb = codebooks["lloyd_beta16" if levels == 16 else "lloyd_beta4"]
    T, H_kv = 300, 8
    k = synth.kv_with_outliers(501, (T, H_kv, 128))
    v = synth.normal_f16(502, (T, H_kv, 128))
    num_slots = 512
    slots = synth.permuted_block_table(503, 1, num_slots)[0][:T].astype(np.int64)
    slots[::17] = -1                      # padding tokens are skipped
    exp = expected_cache(k, v, slots, cb, num_slots, slot_bytes, 0xA5)
    got = run_gpu_encode(gpu, k, v, slots, cb, num_slots, slot_bytes, 0xA5)
    bad = np.argwhere(got != exp)
    assert bad.size == 0, f"{len(bad)} mismatching bytes, first {bad[:5].tolist()}"


@pytest.mark.parametrize("levels,H_kv", [(16, 8), (4, 8), (16, 3)])
def test_encode_separate_codebooks(gpu, codebooks, levels, H_kv):
    """K and V with different codebooks (each role reads its own), and a head
    count that leaves a partial group of vectors in the last wave."""
    print(f"[encode] separate codebooks levels={levels} H_kv={H_kv}", flush=True)
    cb_k = codebooks["lloyd_beta16" if levels == 16 else "lloyd_beta4"]
    cb_v = codebooks["uniform16" if levels == 16 else "uniform4"]
    T = 77
    k = synth.kv_with_outliers(511, (T, H_kv, 128))
    v = synth.normal_f16(512, (T, H_kv, 128))
    slots = np.arange(T, dtype=np.int64)[::-1].copy()
    sb = 144 if levels == 16 else 80
    exp = expected_cache(k, v, slots, cb_k, T, sb, 0x3C, cb_v=cb_v)
    got = run_gpu_encode(gpu, k, v, slots, cb_k, T, sb, 0x3C, cb_v=cb_v)
    bad = np.argwhere(got != exp)
    assert bad.size == 0, f"{len(bad)} mismatching bytes, first {bad[:5].tolist()}"


def test_encode_golden_rows(gpu, golden, codebooks):
    """The fixture rows (outliers + edge rows) through the GPU encoder: equal to
    the checker bit for bit, and equal to the reference's indices."""
    e = golden("encode.npz")
    x = e["x"]                            # (rows, 128)
    rows = x.shape[0]
    for levels, tag in ((16, "k4"), (4, "k2")):
        cb = codebooks["lloyd_beta16" if levels == 16 else "lloyd_beta4"]
        kb = 64 if levels == 16 else 32
        sb = 144 if levels == 16 else 80
        xx = x.reshape(rows, 1, 128)
        got = run_gpu_encode(gpu, xx, xx, np.arange(rows), cb, rows, sb, 0)
        kp, kn, _ = O.encode(x, cb)
        assert np.array_equal(got[:, 0, :kb], kp)
        gn = got[:, 0, 2 * kb:2 * kb + 4].copy().view(np.float32)[:, 0]
        assert np.array_equal(gn.view(np.uint32), kn.view(np.uint32))
        assert np.array_equal(got[:, 0, :kb], e[f"{tag}_idx"])


def test_encode_config2_scale(gpu, codebooks):
    """Config 2: 64 sequences x U[1,256] new tokens scattered into a paged cache."""
    cb = codebooks["lloyd_beta16"]
    rng_lens = (synth._splitmix64(7, 64) % np.uint64(256) + np.uint64(1)).astype(np.int64)
    T = int(rng_lens.sum())
    H_kv = 8
    k = synth.kv_with_outliers(601, (T, H_kv, 128))
    v = synth.normal_f16(602, (T, H_kv, 128))
    num_slots = 64 * 256
    slots = synth.permuted_block_table(603, 1, num_slots)[0][:T].astype(np.int64)
    exp = expected_cache(k, v, slots, cb, num_slots, 144, 0)
    got = run_gpu_encode(gpu, k, v, slots, cb, num_slots, 144, 0)
    assert np.array_equal(got, exp)


def test_encode_golden_rows_wide_batch(gpu, golden, codebooks):
    """The fixture rows repeated into a batch large enough for the 4-lane
    layout (the one config 2 takes): still the reference's indices and norms,
    including the zero, subnormal and fp16-overflow edge rows."""
    e = golden("encode.npz")
    x = e["x"]
    rows = x.shape[0]
    reps = 16
    xx = np.tile(x, (reps, 1)).reshape(rows * reps // 8, 8, 128)
    T = xx.shape[0]
    for levels, tag in ((16, "k4"), (4, "k2")):
        cb = codebooks["lloyd_beta16" if levels == 16 else "lloyd_beta4"]
        kb = 64 if levels == 16 else 32
        sb = 144 if levels == 16 else 80
        print(f"[encode] golden rows x{reps} levels={levels}", flush=True)
        got = run_gpu_encode(gpu, xx, xx, np.arange(T), cb, T, sb, 0)
        codes = got[:, :, :kb].reshape(reps, rows, kb)
        norms = got[:, :, 2 * kb:2 * kb + 4].copy().view(np.float32).reshape(reps, rows)
        for i in range(reps):
            assert np.array_equal(codes[i], e[f"{tag}_idx"])
            assert np.array_equal(norms[i].view(np.uint32), e[f"{tag}_norm"].view(np.uint32))


def test_encode_config0_matches_reference(gpu, golden, codebooks):
    """BASELINE config 0 (4096 tokens x 8 KV heads, outlier K, N(0,1) V): the
    GPU encoder writes exactly the reference's k_idx / v_idx and fp32 norms."""
    import json
    from pathlib import Path
    g = golden("attn_cfg0.npz")
    meta = json.loads((Path(__file__).parent / "golden" / "attn_cfg0.json").read_text())
    N, H_kv, seed = meta["N"], meta["H_kv"], meta["seed"]
    cb = codebooks["lloyd_beta16"]
    k = synth.kv_with_outliers(seed, (1, H_kv, N, 128))[0].transpose(1, 0, 2).copy()
    v = synth.normal_f16(seed + 1, (1, H_kv, N, 128))[0].transpose(1, 0, 2).copy()
    print("[encode] config 0 vs reference", flush=True)
    got = run_gpu_encode(gpu, k, v, np.arange(N), cb, N, 144, 0)
    kidx = got[:, :, :64].transpose(1, 0, 2)
    vidx = got[:, :, 64:128].transpose(1, 0, 2)
    kn = got[:, :, 128:132].copy().view(np.float32)[..., 0].T
    vn = got[:, :, 132:136].copy().view(np.float32)[..., 0].T
    assert np.array_equal(kidx, g["k_idx"][0])
    assert np.array_equal(vidx, g["v_idx"][0])
    assert np.array_equal(kn.view(np.uint32), g["k_norm"][0].view(np.uint32))
    assert np.array_equal(vn.view(np.uint32), g["v_norm"][0].view(np.uint32))


def test_encode_config2_scale_k2v2(gpu, codebooks):
    """Config 2 with the 4-level codebook: 64 sequences x U[1,256] new tokens."""
    cb = codebooks["lloyd_beta4"]
    rng_lens = (synth._splitmix64(8, 64) % np.uint64(256) + np.uint64(1)).astype(np.int64)
    T = int(rng_lens.sum())
    H_kv = 8
    k = synth.kv_with_outliers(611, (T, H_kv, 128))
    v = synth.normal_f16(612, (T, H_kv, 128))
    num_slots = 64 * 256
    slots = synth.permuted_block_table(613, 1, num_slots)[0][:T].astype(np.int64)
    print(f"[encode] config 2 K2V2 T={T}", flush=True)
    exp = expected_cache(k, v, slots, cb, num_slots, 80, 0)
    got = run_gpu_encode(gpu, k, v, slots, cb, num_slots, 80, 0)
    assert np.array_equal(got, exp)
