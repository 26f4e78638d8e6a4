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
