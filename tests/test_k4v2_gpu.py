"""The legacy K4V2 cache (104-byte slots: K 4-bit | V 2-bit | K norm | V norm,
cda_attn_v2.py:29) on the GPU through the C ABI: encode bit-exact against the
checker, the dense loader bit-exact against the checker's decoded rows, and
decode within 2e-3 of the checker on the same cache."""
import numpy as np
import pytest
import torch

from oracle import cda_oracle as O
from oracle import synth

pytestmark = pytest.mark.gpu
TOL = 2e-3


def _t(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _case(seed, seq_lens, H_kv, gs, codebooks, bs=16):
    cbk, cbv = codebooks["lloyd_beta16"], codebooks["lloyd_beta4"]
    B = len(seq_lens)
    N = max(seq_lens)
    k = synth.kv_with_outliers(seed, (B, H_kv, N, 128))
    v = synth.normal_f16(seed + 1, (B, H_kv, N, 128))
    q = synth.normal_f16(seed + 2, (B, H_kv * gs, 128))
    kp, kn, _ = O.encode(k, cbk)
    vp, vn, _ = O.encode(v, cbv)
    W = (N + bs - 1) // bs + 2
    bt = synth.permuted_block_table(seed, B, W)
    cache = O.build_paged_cache(kp, kn, vp, vn, bt, bs, 16, num_blocks=B * W, fill=0xFF, Lv=4)
    sl = np.array(seq_lens, np.int32)
    exp = O.decode_paged(q, cache, bt, sl, cbk, cbv, O.hadamard128(), H_kv=H_kv, block_size=bs)
    return dict(k=k, v=v, q=q, kp=kp, kn=kn, vp=vp, vn=vn, bt=bt, cache=cache, sl=sl, exp=exp,
                cbk=cbk, cbv=cbv, bs=bs)


def test_k4v2_encode_bit_exact(gpu, codebooks):
    from sub0_amd import _native
    cbk, cbv = codebooks["lloyd_beta16"], codebooks["lloyd_beta4"]
    T, H_kv = 300, 8
    k = synth.kv_with_outliers(901, (T, H_kv, 128))
    v = synth.normal_f16(902, (T, H_kv, 128))
    slots = synth.permuted_block_table(903, 1, 512)[0][:T].astype(np.int64)
    slots[::13] = -1
    print("[k4v2] encode", flush=True)
    cache = torch.full((512, H_kv, 104), 0xA5, dtype=torch.uint8, device=gpu)
    _native.paged_encode(_t(k, gpu), _t(v, gpu), _t(slots.astype(np.int32), gpu), cache,
                         _t(cbk, gpu), _t(cbv, gpu))
    torch.cuda.synchronize()
    got = cache.cpu().numpy()
    kp, kn, _ = O.encode(k, cbk)
    vp, vn, _ = O.encode(v, cbv)
    exp = np.full_like(got, 0xA5)
    for t in range(T):
        s = slots[t]
        if s < 0:
            continue
        exp[s, :, :64] = kp[t]
        exp[s, :, 64:96] = vp[t]
        exp[s, :, 96:100] = kn[t].astype(np.float32).view(np.uint8).reshape(H_kv, 4)
        exp[s, :, 100:104] = vn[t].astype(np.float32).view(np.uint8).reshape(H_kv, 4)
    assert np.array_equal(got, exp)


@pytest.mark.parametrize("seq_lens,H_kv,gs", [([700, 33, 1500], 8, 4), ([400, 1], 2, 8)])
def test_k4v2_decode_and_loader(gpu, codebooks, seq_lens, H_kv, gs):
    from sub0_amd import _native
    from sub0_amd.cda.kernels_cuda.hmma_loader import load_decode_hmma, load_fa2_cda_loader
    c = _case(910 + gs, seq_lens, H_kv, gs, codebooks)
    print(f"[k4v2] decode seq_lens={seq_lens} H_kv={H_kv} gs={gs}", flush=True)
    q, cache, bt, sl = _t(c["q"], gpu), _t(c["cache"], gpu), _t(c["bt"], gpu), _t(c["sl"], gpu)
    cbk, cbv = _t(c["cbk"], gpu), _t(c["cbv"], gpu)
    R = _t(O.hadamard128(), gpu)
    out = torch.full_like(q, float("nan"))
    mod = load_decode_hmma(k4v2=True, group_size=gs)
    mod.cda_decode_full_hmma_v3(q, cache, bt, sl, cbk, cbv, R, R.half(), out, gs, c["bs"], 0,
                                max(seq_lens), 1.0 / np.sqrt(128))
    torch.cuda.synchronize()
    o = out.cpu().numpy()
    assert np.isfinite(o).all()
    assert np.abs(o.astype(np.float32) - c["exp"].astype(np.float32)).max() <= TOL
    # dense rotated loader (fa2_cda.py:64-95 with k4v2=True): rows bit-exact
    N = max(seq_lens)
    k_rot, v_rot = load_fa2_cda_loader(k4v2=True).cda_fa2_paged_cache_to_dense_rotated(
        cache, bt, sl, cbk, cbv, c["bs"], N)
    torch.cuda.synchronize()
    kr, vr = k_rot.cpu().numpy(), v_rot.cpu().numpy()
    for b, n in enumerate(seq_lens):
        for h in range(H_kv):
            rows = slice(b * N, b * N + n)
            assert np.array_equal(kr[rows, h].view(np.uint16),
                                  O.decode_rotated(c["kp"][b, h, :n], c["kn"][b, h, :n],
                                                   c["cbk"]).view(np.uint16))
            assert np.array_equal(vr[rows, h].view(np.uint16),
                                  O.decode_rotated(c["vp"][b, h, :n], c["vn"][b, h, :n],
                                                   c["cbv"]).view(np.uint16))
        assert not kr[b * N + n:(b + 1) * N].any()


def test_k4v2_prefill_through_the_dense_bridge(gpu, codebooks):
    """fa2_cda_prefill_varlen_v1(k4v2=True): the K4V2 cache dequantised by the
    K4V2 loader, then the fused attention kernel (fa2_cda.py:98-230 with the
    k4v2 loader of :64-95); against the checker's causal prefill on the same
    cache, 2e-3."""
    from sub0_amd.cda.kernels_cuda.fa2_cda import fa2_cda_prefill_varlen_v1
    seq = [300, 77]
    print(f"[k4v2] prefill seq={seq}", flush=True)
    c = _case(930, seq, 8, 4, codebooks)
    cu = np.concatenate([[0], np.cumsum(seq)]).astype(np.int32)
    q = synth.normal_f16(933, (int(cu[-1]), 32, 128))
    exp = O.prefill_paged(q, cu, c["cache"], c["bt"], c["sl"], c["cbk"], c["cbv"], O.hadamard128(),
                          H_kv=8, block_size=c["bs"])
    qd = _t(q, gpu)
    out = torch.full_like(qd, float("nan"))
    fa2_cda_prefill_varlen_v1(qd, _t(c["cache"], gpu), _t(c["bt"], gpu), _t(cu, gpu),
                              _t(c["sl"], gpu), out, cb_K=_t(c["cbk"], gpu), cb_V=_t(c["cbv"], gpu),
                              rotation_fp32=_t(O.hadamard128(), gpu), group_size=4,
                              block_size=c["bs"], max_query_len=300, max_seq_len=300, k4v2=True)
    torch.cuda.synchronize()
    o = out.cpu().numpy()
    assert np.isfinite(o).all()
    assert np.abs(o.astype(np.float32) - exp.astype(np.float32)).max() <= TOL
