"""Parity at the benchmark's full sizes, against plain PyTorch references on
the GPU built from the dense dequantised cache (paged_to_dense, itself
bit-exact against the checker): the BASELINE config-1 headline cell
(B=32, N=65536) for decode on both split kernels (and K2V2 on the
page-streaming kernel), and the config-3 draw for prefill.  The references follow the checker's arithmetic: q_rot rounded to
fp16, scores/softmax/PV in float64 (decode) or float32 (prefill) on the fp16
K/V rows, O_rot rounded to fp16, then the inverse rotation rounded to fp16."""
import pytest
import torch

pytestmark = pytest.mark.gpu
TOL = 2e-3
H_Q, H_KV, D, BS = 32, 8, 128, 16


def _decode_reference(w, k_rot, v_rot):
    R = w["R"].double()
    q_rot = (w["q"].double() @ R).float().half().double()          # (B, 32, 128)
    B, N = w["B"], w["N"]
    out = torch.empty(B, H_Q, D, dtype=torch.float16, device=w["q"].device)
    for b in range(B):
        K = k_rot[b * N:(b + 1) * N].double()                      # (N, 8, 128)
        V = v_rot[b * N:(b + 1) * N].double()
        for h in range(H_KV):
            qh = q_rot[b, 4 * h:4 * h + 4]                          # (4, 128)
            s = (qh @ K[:, h].T) / D ** 0.5                         # (4, N)
            p = torch.softmax(s, dim=-1)
            o_rot = (p @ V[:, h]).float().half().double()
            out[b, 4 * h:4 * h + 4] = (o_rot @ R.T).float().half()
    return out


@pytest.mark.parametrize("stream", [True, False], ids=["stream", "general"])
def test_decode_fullsize_against_torch(gpu, stream):
    import bench
    from sub0_amd import _native
    print(f"[fullsize] decode B=32 N=65536 stream={stream}", flush=True)
    w = bench.make_workload(32, 65536, gpu)
    k_rot, v_rot = _native.paged_to_dense(w["cache"], w["bt"], w["seq"], w["cb"], w["cb"],
                                          block_size=BS, max_seq_len=w["N"])
    ref = _decode_reference(w, k_rot, v_rot)
    del k_rot, v_rot
    _native.set_stream_kernel(stream)
    try:
        bench.decode_call(w)()
        torch.cuda.synchronize()
    finally:
        _native.set_stream_kernel(True)
    out = w["out"]
    assert torch.isfinite(out).all()
    err = (out.float() - ref.float()).abs().max().item()
    print(f"[fullsize] decode max abs err {err:.3e}", flush=True)
    assert err <= TOL


@pytest.mark.parametrize("B,N", [(2, 131072), (1, 262144)], ids=["B2_N128K", "B1_N256K"])
def test_decode_long_context_against_torch(gpu, B, N):
    """Contexts past the metric grid: 128K (the reference's longest
    throughput cell, Fig. 2 / Table A3) and 256K tokens per sequence, through
    the page-streaming kernel with the default split plan."""
    import bench
    from sub0_amd import _native
    print(f"[fullsize] decode B={B} N={N}", flush=True)
    w = bench.make_workload(B, N, gpu)
    k_rot, v_rot = _native.paged_to_dense(w["cache"], w["bt"], w["seq"], w["cb"], w["cb"],
                                          block_size=BS, max_seq_len=w["N"])
    ref = _decode_reference(w, k_rot, v_rot)
    del k_rot, v_rot
    bench.decode_call(w)()
    torch.cuda.synchronize()
    out = w["out"]
    assert torch.isfinite(out).all()
    err = (out.float() - ref.float()).abs().max().item()
    print(f"[fullsize] decode B={B} N={N} max abs err {err:.3e}", flush=True)
    assert err <= TOL


def _k2v2_dense(w, b):
    """Rows of sequence b of a K2V2 cache (80-byte slots: 32 K code bytes, 32 V
    code bytes, fp32 Kn, fp32 Vn) decoded as fp16(centroid * norm), dim 4j in
    bits 7:6 of byte j (compression.py:355-359, 375-397)."""
    N = w["N"]
    t = torch.arange(N, device=w["q"].device)
    slots = w["bt"][b, t // BS].long() * BS + t % BS
    rows = w["cache"][slots]                                        # (N, 8, 80) u8
    shifts = torch.tensor([6, 4, 2, 0], device=rows.device, dtype=torch.uint8)

    def unpack(x):                                                  # (N, 8, 32) -> (N, 8, 128)
        return ((x.unsqueeze(-1) >> shifts) & 3).reshape(*x.shape[:-1], 128).long()

    kn = rows[..., 64:68].contiguous().view(torch.float32)          # (N, 8, 1)
    vn = rows[..., 68:72].contiguous().view(torch.float32)
    cb = w["cb"].float()
    K = (cb[unpack(rows[..., :32])] * kn).half()
    V = (cb[unpack(rows[..., 32:64])] * vn).half()
    return K, V


def test_decode_k2v2_fullsize_against_torch(gpu):
    """K2V2 (4-level codebook, 80-byte slots) at B=32, N=65536 on the
    page-streaming kernel."""
    import bench
    print("[fullsize] K2V2 decode B=32 N=65536", flush=True)
    w = bench.make_workload(32, 65536, gpu, levels=4)
    assert w["cache"].shape[-1] == 80
    bench.decode_call(w)()
    torch.cuda.synchronize()
    R = w["R"].double()
    q_rot = (w["q"].double() @ R).float().half().double()
    ref = torch.empty_like(w["out"])
    for b in range(w["B"]):
        K, V = _k2v2_dense(w, b)
        for h in range(H_KV):
            qh = q_rot[b, 4 * h:4 * h + 4]
            s = (qh @ K[:, h].double().T) / D ** 0.5
            p = torch.softmax(s, dim=-1)
            o_rot = (p @ V[:, h].double()).float().half().double()
            ref[b, 4 * h:4 * h + 4] = (o_rot @ R.T).float().half()
    out = w["out"]
    assert torch.isfinite(out).all()
    err = (out.float() - ref.float()).abs().max().item()
    print(f"[fullsize] K2V2 decode max abs err {err:.3e}", flush=True)
    assert err <= TOL


@pytest.mark.parametrize("source", ["compressed", "dense"])
def test_prefill_fullsize_against_torch(gpu, source):
    import bench
    from sub0_amd import _native
    print(f"[fullsize] prefill config 3 (8 sequences, 512-8192 tokens) source={source}",
          flush=True)
    w = bench.make_prefill_workload(gpu)
    bench.prefill_call(w, source)()
    torch.cuda.synchronize()
    out = w["out"]
    assert torch.isfinite(out).all()
    lens = w["lens"]
    L = max(lens)
    k_rot, v_rot = _native.paged_to_dense(w["cache"], w["bt"], w["seq"], w["cb"], w["cb"],
                                          block_size=BS, max_seq_len=L)
    R = w["R"].float()
    worst = 0.0
    t0 = 0
    for i, n in enumerate(lens):
        q = w["q"][t0:t0 + n]                                       # (n, 32, 128)
        q_rot = (q.float() @ R).half().float()
        K = k_rot[i * L:i * L + n].float()
        V = v_rot[i * L:i * L + n].float()
        mask = torch.ones(n, n, dtype=torch.bool, device=gpu).tril()
        for h in range(H_KV):
            qh = q_rot[:, 4 * h:4 * h + 4].transpose(0, 1)          # (4, n, 128)
            s = (qh @ K[:, h].T) / D ** 0.5                         # (4, n, n)
            s = s.masked_fill(~mask, float("-inf"))
            p = torch.softmax(s, dim=-1)
            o_rot = (p @ V[:, h]).half().float()                    # (4, n, 128)
            ref = (o_rot @ R.T).half()
            got = out[t0:t0 + n, 4 * h:4 * h + 4].transpose(0, 1)
            worst = max(worst, (got.float() - ref.float()).abs().max().item())
            del s, p
        t0 += n
    print(f"[fullsize] prefill max abs err {worst:.3e}", flush=True)
    assert worst <= TOL
