"""The config-4 decode loop (bench.py --e2e) at a tiny shape: a Mistral-style
decoder driven through the cda_v2 backend, prefill then greedy decode as graph
replays that advance their own state.  The replayed steps must produce the
same tokens as eager steps from the same state (deterministic kernels, and
the captured metadata buffers are the ones the replays update)."""
import pytest
import torch

pytestmark = pytest.mark.gpu


def test_e2e_replays_match_eager_steps(gpu):
    import bench
    print("[e2e] B=3 prefix=40 steps=6 layers=2 heads=8/2", flush=True)
    r = bench.e2e_run(gpu, B=3, prefix=40, steps=6, layers=2, heads=8, kv_heads=2, ffn=512,
                      vocab=500, check_eager=3)
    assert len(r["eager_tokens"]) == 3
    for i, want in enumerate(r["eager_tokens"]):
        got = r["produced"][2 + i]
        assert torch.equal(got, want), f"replay {i + 1}: {got.tolist()} != {want.tolist()}"
    assert r["tokens_per_s"] > 0 and r["attn_ms"] > 0


def test_e2e_gs8_heads(gpu):
    """GQA group of 8 (16 Q / 2 KV heads) through the same loop."""
    import bench
    print("[e2e] gs8 B=2 prefix=70", flush=True)
    r = bench.e2e_run(gpu, B=2, prefix=70, steps=4, layers=1, heads=16, kv_heads=2, ffn=256,
                      vocab=300, check_eager=2)
    for i, want in enumerate(r["eager_tokens"]):
        assert torch.equal(r["produced"][2 + i], want)


def test_e2e_config4_full_size(gpu):
    """BASELINE config 4 at its stated shape: 32 layers, hidden 4096, 32/8
    heads, SwiGLU 14336, 32 sequences x 16384-token prefix, K4V4 cache, 256
    greedy steps (the whole config).  Prints and checks the run's decode
    tokens/s and attention share; replayed steps produce the eager steps'
    tokens, and one layer's decode over its ~16.6K-token cache is within 2e-3
    of a float64 torch reference on the dense dequantised rows of that cache."""
    import bench
    from sub0_amd import _native
    steps = 256
    print(f"[e2e] config 4: B=32 prefix=16384 steps={steps} layers=32", flush=True)
    r = bench.e2e_run(gpu, B=32, prefix=16384, steps=steps, check_eager=3, keep_state=True)
    share = r["attn_ms"] / r["step_ms"]
    print(f"[e2e] config 4: {r['tokens_per_s']:.1f} tokens/s over {r['decode_steps']} decode "
          f"steps, {r['step_ms']:.3f} ms per step, attention (cache update + attention, "
          f"32 layers) {r['attn_ms']:.3f} ms = {share:.3f} of the step; prefill "
          f"{r['prefill_s']:.2f} s", flush=True)
    assert r["decode_steps"] >= steps - 1 and r["tokens_per_s"] > 0
    assert 0.0 < share < 1.0
    for i, want in enumerate(r["eager_tokens"]):
        assert torch.equal(r["produced"][2 + i], want), f"replay {i + 1}"
    m, caches, bt = r["model"], r["caches"], r["block_table"]
    lens = r["cached_lens"].to(torch.int32)
    N = int(lens[0])
    assert bool((lens == N).all()) and N == 16384 + steps
    li = 17
    A = m.A
    B, H, Hkv, D = 32, 32, 8, 128
    g = torch.Generator(device=gpu).manual_seed(5)
    q = torch.randn(B, H, D, generator=g, device=gpu, dtype=torch.float16)
    md = A.CDAv2AttentionMetadata(
        num_actual_tokens=B, num_reqs=B, max_query_len=1, max_seq_len=N,
        query_start_loc=torch.arange(B + 1, dtype=torch.int32, device=gpu),
        seq_lens=lens, block_table=bt,
        slot_mapping=torch.zeros(B, dtype=torch.int64, device=gpu))
    out = torch.empty(B, H * D, dtype=torch.float16, device=gpu)
    m.impl.forward(None, q, q[:, :Hkv], q[:, :Hkv], caches[li], md, out)
    torch.cuda.synchronize()
    kv = A._as_uint8_cache(caches[li]).reshape(-1, Hkv, 144)
    cb, _, R, _ = A._get_hmma_artifacts(*A._get_compressors(gpu), gpu)
    k_rot, v_rot = _native.paged_to_dense(kv, bt, lens, cb, cb, block_size=16, max_seq_len=N)
    q_rot = (q.double() @ R.double()).float().half().double()
    ref = torch.empty(B, H, D, dtype=torch.float16, device=gpu)
    for b in range(B):
        K = k_rot[b * N:(b + 1) * N].double()
        V = v_rot[b * N:(b + 1) * N].double()
        for h in range(Hkv):
            s = (q_rot[b, 4 * h:4 * h + 4] @ K[:, h].T) / D ** 0.5
            o_rot = (torch.softmax(s, dim=-1) @ V[:, h]).float().half().double()
            ref[b, 4 * h:4 * h + 4] = (o_rot @ R.double().T).float().half()
    err = (out.view(B, H, D).float() - ref.float()).abs().max().item()
    print(f"[e2e] config 4 layer {li} decode max abs err {err:.3e}", flush=True)
    assert err <= 2e-3

