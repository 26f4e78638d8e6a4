"""The torch.ops boundary on the GPU: torch.ops.cda_hip.decode inside a
captured HIP graph (every replay against the checker, eager work between
replays), and the FA2-fork comparator namespace torch.ops._cda_vllm_fa2_fork_C
(dequantize_compressed_kv bit-exact against the checker's decoded rows; the
varlen forwards within 2e-3 of an fp32 torch reference of the same rotated-
frame attention over those rows)."""
import numpy as np
import pytest
import torch

from oracle import cda_oracle as O
from oracle import synth
from tests.cases import make_decode_case

pytestmark = pytest.mark.gpu
TOL = 2e-3


def _t(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def test_decode_through_torch_ops_in_graph(gpu):
    from sub0_amd.cda._prebuilt_loader import load_torch_ops_library
    ops = load_torch_ops_library("cda_hip")
    print("[torch-ops] decode in a captured graph", flush=True)
    case = make_decode_case(8100, [1500, 77, 3000], H_kv=8, gs=4, fill=0xFF)
    q, cache, bt, sl = (_t(case.q, gpu), _t(case.cache, gpu), _t(case.block_table, gpu),
                        _t(case.seq_lens, gpu))
    cb, R = _t(case.cb_k, gpu), _t(case.R, gpu)
    out = torch.full_like(q, float("nan"))
    args = (q, cache, bt, sl, cb, cb, R, R.half(), out, 4, 16, 0, 3000, float(1 / np.sqrt(128)))
    ops.decode(*args)                      # eager (also warms up the codebook cache)
    torch.cuda.synchronize()
    eager = out.cpu().numpy()
    assert np.abs(eager.astype(np.float32) - case.expected.astype(np.float32)).max() <= TOL
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            ops.decode(*args)
    torch.cuda.current_stream().wait_stream(s)
    for i in range(3):
        out.fill_(float("nan"))
        _ = (q.float() * 2).sum()          # unrelated eager work between replays
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(out.cpu().numpy().view(np.uint16), eager.view(np.uint16)), i


def _rows(seed, lens, H_kv, cb):
    """Encoded rows of several sequences, flattened B-major (total_k, H_kv, .)."""
    k = synth.kv_with_outliers(seed, (sum(lens), H_kv, 128))
    v = synth.normal_f16(seed + 1, (sum(lens), H_kv, 128))
    kp, kn, _ = O.encode(k, cb)
    vp, vn, _ = O.encode(v, cb)
    return kp, kn, vp, vn


def _attn_ref(q, k, v, cu_q, lens, scale, causal):
    """fp32 torch attention per sequence, rotated frame, fp16 out."""
    out = torch.empty_like(q)
    H_q, H_kv = q.shape[1], k.shape[1]
    g = H_q // H_kv
    k0 = 0
    for b, L in enumerate(lens):
        qs = q[cu_q[b]:cu_q[b + 1]].float()                 # (M, H_q, D)
        ks = k[k0:k0 + L].float().repeat_interleave(g, dim=1)
        vs = v[k0:k0 + L].float().repeat_interleave(g, dim=1)
        s = torch.einsum("mhd,khd->hmk", qs, ks) * scale
        if causal:
            M = qs.shape[0]
            mask = torch.arange(L, device=q.device)[None, :] <= (
                torch.arange(M, device=q.device)[:, None] + L - M)
            s = s.masked_fill(~mask[None], float("-inf"))
        p = torch.softmax(s, dim=-1)
        out[cu_q[b]:cu_q[b + 1]] = torch.einsum("hmk,khd->mhd", p, vs).half()
        k0 += L
    return out


def test_fork_dequantize_bit_exact(gpu, codebooks):
    from sub0_amd.cda._prebuilt_loader import load_torch_ops_library
    fork = load_torch_ops_library("_cda_vllm_fa2_fork_C")
    cb = codebooks["lloyd_beta16"]
    kp, kn, vp, vn = _rows(8200, [300, 41], 8, cb)
    print("[torch-ops] fork dequantize_compressed_kv", flush=True)
    k, v = fork.dequantize_compressed_kv(_t(kp, gpu), _t(kn, gpu), _t(vp, gpu), _t(vn, gpu),
                                         _t(cb, gpu), _t(cb, gpu))
    torch.cuda.synchronize()
    assert np.array_equal(k.cpu().numpy().view(np.uint16),
                          O.decode_rotated(kp, kn, cb).view(np.uint16))
    assert np.array_equal(v.cpu().numpy().view(np.uint16),
                          O.decode_rotated(vp, vn, cb).view(np.uint16))


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("paged", [False, True])
def test_fork_varlen_compressed(gpu, codebooks, causal, paged):
    from sub0_amd.cda._prebuilt_loader import load_torch_ops_library
    fork = load_torch_ops_library("_cda_vllm_fa2_fork_C")
    cb = codebooks["lloyd_beta16"]
    lens, qlens, H_kv, H_q = [300, 97, 1000], [37, 1, 64], 8, 32
    kp, kn, vp, vn = _rows(8300, lens, H_kv, cb)
    q = _t(synth.normal_f16(8303, (sum(qlens), H_q, 128)), gpu)
    cu_q = torch.tensor(np.concatenate([[0], np.cumsum(qlens)]), dtype=torch.int32, device=gpu)
    cu_k = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int32, device=gpu)
    scale = float(1 / np.sqrt(128))
    kd = _t(O.decode_rotated(kp, kn, cb), gpu)
    vd = _t(O.decode_rotated(vp, vn, cb), gpu)
    ref = _attn_ref(q, kd, vd, cu_q.tolist(), lens, scale, causal)
    print(f"[torch-ops] fork varlen compressed causal={causal} paged={paged}", flush=True)
    out = torch.full_like(q, float("nan"))
    tail = (max(qlens), max(lens), 0.0, scale, False, causal, -1, -1, 0.0, False, 0)
    if not paged:
        r = fork.varlen_fwd_compressed_kv(q, _t(kp, gpu), _t(kn, gpu), _t(vp, gpu), _t(vn, gpu),
                                          _t(cb, gpu), _t(cb, gpu), out, cu_q, cu_k, None,
                                          *tail, None)
    else:
        # paged pools (num_blocks, 16, H_kv, 64): scatter rows through a permuted table
        bs, W = 16, (max(lens) + 15) // 16
        bt = synth.permuted_block_table(8304, len(lens), W)
        nb = len(lens) * W
        pools = [np.zeros((nb * bs,) + a.shape[1:], a.dtype) for a in (kp, kn, vp, vn)]
        k0 = 0
        for b, L in enumerate(lens):
            t = np.arange(L)
            slots = bt[b][t // bs] * bs + t % bs
            for pool, a in zip(pools, (kp, kn, vp, vn)):
                pool[slots] = a[k0:k0 + L]
            k0 += L
        kpp, knp, vpp, vnp = (_t(p.reshape((nb, bs) + p.shape[1:]), gpu) for p in pools)
        r = fork.varlen_fwd_compressed_kv_fused(
            q, kpp, knp, vpp, vnp, _t(cb, gpu), _t(cb, gpu), out, cu_q, None,
            torch.tensor(lens, dtype=torch.int32, device=gpu), _t(bt, gpu), None, *tail,
            False, None)
    torch.cuda.synchronize()
    assert r[0] is out
    err = float((out.float() - ref.float()).abs().max())
    assert err <= TOL, err


@pytest.mark.parametrize("entry", ["dense", "two_step_4d", "fused_paged"])
def test_fork_python_interface(gpu, codebooks, entry):
    """The Python entry points of kernels_vllm_fa2_fork (interface.py of the
    reference): dense varlen, the two-step bridge on the compressor's
    (B, H_kv, N, 64) layout, and the fused call on paged pools."""
    from sub0_amd.cda import kernels_vllm_fa2_fork as F
    cb = codebooks["lloyd_beta16"]
    H_kv, H_q = 8, 32
    lens = [256, 256] if entry == "two_step_4d" else [300, 97, 1000]
    qlens = [16, 64] if entry == "two_step_4d" else [37, 1, 64]
    kp, kn, vp, vn = _rows(8400, lens, H_kv, cb)
    q = _t(synth.normal_f16(8403, (sum(qlens), H_q, 128)), gpu)
    cu_q = torch.tensor(np.concatenate([[0], np.cumsum(qlens)]), dtype=torch.int32, device=gpu)
    cu_k = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int32, device=gpu)
    kd = _t(O.decode_rotated(kp, kn, cb), gpu)
    vd = _t(O.decode_rotated(vp, vn, cb), gpu)
    ref = _attn_ref(q, kd, vd, cu_q.tolist(), lens, float(1 / np.sqrt(128)), True)
    cbt = _t(cb, gpu)
    print(f"[torch-ops] fork python interface {entry}", flush=True)
    if entry == "dense":
        out = F.flash_attn_varlen_func(q, kd, vd, max(qlens), cu_q, max(lens),
                                       cu_seqlens_k=cu_k, causal=True)
    elif entry == "two_step_4d":
        B, N = len(lens), lens[0]

        def slot(a):                      # (B*N, H_kv, .) -> (B, H_kv, N, .)
            return _t(a.reshape((B, N) + a.shape[1:]).swapaxes(1, 2), gpu)
        out = F.flash_attn_varlen_compressed_kv_func(
            q, slot(kp), slot(kn), slot(vp), slot(vn), cbt, cbt, max(qlens), cu_q, N, cu_k,
            causal=True)
    else:
        bs, W = 16, (max(lens) + 15) // 16
        bt = synth.permuted_block_table(8404, len(lens), W)
        nb = len(lens) * W
        pools = [np.zeros((nb * bs,) + a.shape[1:], a.dtype) for a in (kp, kn, vp, vn)]
        k0 = 0
        for b, L in enumerate(lens):
            t = np.arange(L)
            slots = bt[b][t // bs] * bs + t % bs
            for pool, a in zip(pools, (kp, kn, vp, vn)):
                pool[slots] = a[k0:k0 + L]
            k0 += L
        kpp, knp, vpp, vnp = (_t(p.reshape((nb, bs) + p.shape[1:]), gpu) for p in pools)
        out = F.flash_attn_varlen_compressed_kv_fused_func(
            q, kpp, knp, vpp, vnp, cbt, cbt, max(qlens), cu_q, max(lens),
            seqused_k=torch.tensor(lens, dtype=torch.int32, device=gpu), block_table=_t(bt, gpu),
            causal=True)
    torch.cuda.synchronize()
    err = float((out.float() - ref.float()).abs().max())
    assert err <= TOL, err


def test_native_ops_error_types(gpu):
    """The C++ registrations raise the reference wrappers' exception types
    (wrappers.py:110-113, 143-148) before launching anything: TypeError for
    dtypes, ValueError for shapes, NotImplementedError for fork features the
    kernels lack."""
    from sub0_amd.cda._prebuilt_loader import load_torch_ops_library
    ops = load_torch_ops_library("cda_hip")
    fork = load_torch_ops_library("_cda_vllm_fa2_fork_C")
    q = torch.zeros(2, 32, 128, dtype=torch.float16, device=gpu)
    kv = torch.zeros(64, 8, 144, dtype=torch.uint8, device=gpu)
    bt = torch.zeros(2, 4, dtype=torch.int32, device=gpu)
    sl = torch.full((2,), 40, dtype=torch.int32, device=gpu)
    cb = torch.zeros(16, device=gpu)
    R = torch.eye(128, device=gpu)
    out = torch.empty_like(q)
    with pytest.raises(TypeError):
        ops.decode(q.float(), kv, bt, sl, cb, cb, R, R.half(), out, 4, 16, 0, 40, 0.1)
    with pytest.raises(TypeError):
        ops.decode(q, kv, bt.long(), sl, cb, cb, R, R.half(), out, 4, 16, 0, 40, 0.1)
    with pytest.raises(ValueError):
        ops.decode(q[:, :, :64].contiguous(), kv, bt, sl, cb, cb, R, R.half(), out, 4, 16, 0,
                   40, 0.1)
    with pytest.raises(ValueError):
        ops.decode(q, kv, bt, sl, cb, cb, R, R.half(), out.cpu(), 4, 16, 0, 40, 0.1)
    k = torch.zeros(3, 8, 128, dtype=torch.float16, device=gpu)
    with pytest.raises(TypeError):
        ops.encode(k.float(), k.float(), torch.zeros(3, dtype=torch.int32, device=gpu), kv, cb, cb)
    with pytest.raises(ValueError):
        ops.encode(k[:, :, :64].contiguous(), k[:, :, :64].contiguous(),
                   torch.zeros(3, dtype=torch.int32, device=gpu), kv, cb, cb)
    cu = torch.tensor([0, 3], dtype=torch.int32, device=gpu)
    with pytest.raises(NotImplementedError):
        fork.varlen_fwd(k, k, k, None, cu, cu, None, None, None, None, 3, 3, 0.1, 0.1, False,
                        True, -1, -1, 0.0, False, 1, None)
    torch.cuda.synchronize()


@pytest.mark.parametrize("causal,scale", [(True, None), (False, None), (False, -0.05)])
def test_fork_softmax_lse(gpu, causal, scale):
    """return_softmax_lse=True (reference interface.py:234-258): out and the
    (H_q, total_q) fp32 softmax_lse = log(sum exp(scale * q.k)) over each
    query's visible keys, against fp32 torch.logsumexp; a sequence with more
    queries than keys leaves its first causal rows with no visible key, which
    get out = 0 and lse = +inf (FlashAttention-2's convention).  Tolerance
    1e-3 on lse: the kernel sums the fp16-rounded weights (relative error
    <= 2^-11 per term, <= 5e-4 after the log)."""
    from sub0_amd.cda import kernels_vllm_fa2_fork as F
    H_kv, H_q = 8, 32
    lens, qlens = [300, 97, 1000, 20], [37, 1, 64, 40]
    q = _t(synth.normal_f16(8500, (sum(qlens), H_q, 128)), gpu)
    k = _t(synth.normal_f16(8501, (sum(lens), H_kv, 128)), gpu)
    v = _t(synth.normal_f16(8502, (sum(lens), H_kv, 128)), gpu)
    cu_q = torch.tensor(np.concatenate([[0], np.cumsum(qlens)]), dtype=torch.int32, device=gpu)
    cu_k = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int32, device=gpu)
    sc = float(1 / np.sqrt(128)) if scale is None else scale
    print(f"[torch-ops] fork softmax_lse causal={causal} scale={sc}", flush=True)
    out, lse = F.flash_attn_varlen_func(q, k, v, max(qlens), cu_q, max(lens), cu_seqlens_k=cu_k,
                                        causal=causal, softmax_scale=scale,
                                        return_softmax_lse=True)
    torch.cuda.synchronize()
    assert tuple(lse.shape) == (H_q, sum(qlens)) and lse.dtype == torch.float32
    ref_out = torch.zeros_like(q, dtype=torch.float32)
    ref_lse = torch.empty(H_q, sum(qlens), dtype=torch.float32, device=gpu)
    g = H_q // H_kv
    cq = cu_q.tolist()
    k0 = 0
    for b, L in enumerate(lens):
        qs = q[cq[b]:cq[b + 1]].float()
        ks = k[k0:k0 + L].float().repeat_interleave(g, dim=1)
        vs = v[k0:k0 + L].float().repeat_interleave(g, dim=1)
        s = torch.einsum("mhd,khd->hmk", qs, ks) * sc
        if causal:
            M = qs.shape[0]
            mask = torch.arange(L, device=gpu)[None, :] <= (
                torch.arange(M, device=gpu)[:, None] + L - M)
            s = s.masked_fill(~mask[None], float("-inf"))
        lb = torch.logsumexp(s, dim=-1)                          # (H_q, M)
        empty = torch.isinf(lb) & (lb < 0)
        p = torch.softmax(s, dim=-1).nan_to_num(0.0)
        ref_out[cq[b]:cq[b + 1]] = torch.einsum("hmk,khd->mhd", p, vs)
        ref_lse[:, cq[b]:cq[b + 1]] = torch.where(empty, torch.full_like(lb, float("inf")), lb)
        k0 += L
    fin = torch.isfinite(ref_lse)
    assert torch.equal(fin, torch.isfinite(lse)), "rows with no visible key must read +inf"
    assert bool((lse[~fin] == float("inf")).all())
    assert (int((~fin).sum()) > 0) == causal
    err_lse = float((lse[fin] - ref_lse[fin]).abs().max())
    err_out = float((out.float() - ref_out).abs().max())
    assert err_lse <= 1e-3, err_lse
    assert err_out <= TOL, err_out
