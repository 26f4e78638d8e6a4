"""GPU parity of the vLLM backend glue (cda_attn_v2.py:655-748, 760-836,
1301-1328, 1565-1695) driven with stand-in metadata, as vLLM would drive it
for three requests: a prefill step, a decode step, then a mixed step (two
decodes and one chunked-prefill continuation).  Each step's cache update is
checked bit-exact against the checker's encode (payload bytes 0..135) and
its attention output against the checker's prefill / decode on the cache the
GPU wrote, to 2e-3 max-abs."""
import numpy as np
import pytest
import torch

from oracle import cda_oracle as O
from oracle import synth

pytestmark = pytest.mark.gpu
TOL = 2e-3
H_Q, H_KV, D, BS = 32, 8, 128, 16


class Scenario:
    """Three requests over one fp16-typed vLLM cache (nb, 16, 8, 72)."""

    def __init__(self, dev, seed=77, fill=0x5A, nmax=160):
        from sub0_amd.cda.kernels_cuda.vllm_integration import cda_attn_v2 as A
        self.A = A
        self.dev = dev
        Impl = A.get_backend_classes()[1]
        self.impl = Impl(H_Q, D, 1.0 / np.sqrt(D), num_kv_heads=H_KV)
        self.nmax = nmax
        self.W = (self.nmax + BS - 1) // BS + 1
        self.B = 3
        self.bt = synth.permuted_block_table(seed, self.B, self.W)
        self.k = synth.kv_with_outliers(seed, (self.B, self.nmax, H_KV, D))
        self.v = synth.normal_f16(seed + 1, (self.B, self.nmax, H_KV, D))
        self.q = synth.normal_f16(seed + 2, (self.B, self.nmax, H_Q, D))
        nb = self.B * self.W
        self.cache = torch.full((nb, BS, H_KV, 72), 0, dtype=torch.float16, device=dev)
        self.cache.view(torch.uint8).fill_(fill)
        self.lens = np.zeros(self.B, dtype=np.int32)
        self.cb = A._get_compressors(dev)[0].codebook.cpu().numpy()

    def slots(self, b, t0, t1):
        t = np.arange(t0, t1)
        return self.bt[b, t // BS].astype(np.int64) * BS + t % BS

    def step(self, new, out2d=False):
        """Append ``new[b]`` tokens to each request; run update + forward.
        Returns (output (T, H_q, D) fp16 numpy, per-request query ranges)."""
        dev = self.dev
        rows_k, rows_v, rows_q, slots, cu = [], [], [], [], [0]
        for b, n in enumerate(new):
            t0, t1 = self.lens[b], self.lens[b] + n
            rows_k.append(self.k[b, t0:t1])
            rows_v.append(self.v[b, t0:t1])
            rows_q.append(self.q[b, t0:t1])
            slots.append(self.slots(b, t0, t1))
            cu.append(cu[-1] + n)
        self.lens += np.asarray(new, dtype=np.int32)
        K = np.concatenate(rows_k)
        V = np.concatenate(rows_v)
        self.last_kv = (K, V)
        Q = np.concatenate(rows_q)
        sm = np.concatenate(slots)
        T = len(sm)
        t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
        self.impl.do_kv_cache_update(None, t(K), t(V), self.cache, t(sm.astype(np.int64)))
        md = self.A.CDAv2AttentionMetadata(
            num_actual_tokens=T, num_reqs=self.B, max_query_len=int(max(new)),
            max_seq_len=int(self.lens.max()), query_start_loc=t(np.asarray(cu, np.int32)),
            seq_lens=t(self.lens), block_table=t(self.bt), slot_mapping=t(sm))
        out = torch.full((T, H_Q * D) if out2d else (T, H_Q, D), float("nan"),
                         dtype=torch.float16, device=dev)
        self.impl.forward(None, t(Q), t(K), t(V), self.cache, md, out)
        torch.cuda.synchronize()
        # cache bytes of this step's tokens against the checker's encode
        got = self.cache.view(torch.uint8).view(-1, H_KV, 144).cpu().numpy()
        kp, kn, _ = O.encode(K, self.cb)
        vp, vn, _ = O.encode(V, self.cb)
        exp = np.concatenate([kp, vp, kn[..., None].view(np.uint8),
                              vn[..., None].view(np.uint8)], axis=-1)
        assert np.array_equal(got[sm, :, :136], exp), "cache update differs from the checker"
        return out.view(T, H_Q, D).cpu().numpy(), got, Q, cu

    def expected_prefill(self, cache, Q, cu, reqs):
        """Checker prefill of the given requests' query rows."""
        sel_q = np.concatenate([Q[cu[b]:cu[b + 1]] for b in reqs])
        qlens = [cu[b + 1] - cu[b] for b in reqs]
        cu_r = np.concatenate([[0], np.cumsum(qlens)]).astype(np.int32)
        return O.prefill_paged(sel_q, cu_r, cache, self.bt[reqs], self.lens[reqs], self.cb,
                               self.cb, O.hadamard128(), H_kv=H_KV, block_size=BS)

    def expected_decode(self, cache, Q, cu, reqs):
        q = np.stack([Q[cu[b]] for b in reqs])
        return O.decode_paged(q, cache, self.bt[reqs], self.lens[reqs], self.cb, self.cb,
                              O.hadamard128(), H_kv=H_KV, block_size=BS)


def check(out, exp, tol=TOL):
    assert np.isfinite(out).all(), "non-finite output"
    err = float(np.abs(out.astype(np.float32) - exp.astype(np.float32)).max())
    assert err <= tol, f"max abs err {err}"
    return err


def test_backend_prefill_decode_mixed(gpu):
    sc = Scenario(gpu)
    print("[backend] prefill step lens=[37,100,64]", flush=True)
    out, cache, Q, cu = sc.step([37, 100, 64])
    check(out, sc.expected_prefill(cache, Q, cu, [0, 1, 2]))

    print("[backend] decode step (2-D output buffer)", flush=True)
    out, cache, Q, cu = sc.step([1, 1, 1], out2d=True)
    check(out, sc.expected_decode(cache, Q, cu, [0, 1, 2]))

    print("[backend] mixed step: two decodes + 20-token chunk", flush=True)
    out, cache, Q, cu = sc.step([1, 1, 20])
    check(out[:2], sc.expected_decode(cache, Q, cu, [0, 1]))
    check(out[2:], sc.expected_prefill(cache, Q, cu, [2]))


def test_backend_decode_graph_replay(gpu):
    """A captured decode forward replays to the eager result every time."""
    sc = Scenario(gpu, seed=78)
    sc.step([90, 33, 150])
    out, cache, Q, cu = sc.step([1, 1, 1])
    check(out, sc.expected_decode(cache, Q, cu, [0, 1, 2]))
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(gpu)
    q = t(np.stack([Q[i] for i in range(3)]))
    md = sc.A.CDAv2AttentionMetadata(
        num_actual_tokens=3, num_reqs=3, max_query_len=1, max_seq_len=int(sc.lens.max()),
        query_start_loc=t(np.arange(4, dtype=np.int32)), seq_lens=t(sc.lens),
        block_table=t(sc.bt), slot_mapping=t(np.zeros(3, np.int64)))
    o = torch.empty(3, H_Q, D, dtype=torch.float16, device=gpu)

    def call():
        sc.impl.forward(None, q, None, None, sc.cache, md, o)

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(3):
            call()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    eager = o.clone()
    check(eager.cpu().numpy(), out)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        call()
    for _ in range(3):
        o.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(o, eager)


def test_backend_long_prefill_takes_dense_bridge(gpu, monkeypatch):
    """A prefill step with a 300-token request (max_query_len >= 256: the
    wrapper's default source is the dense bridge) and a follow-up decode."""
    from sub0_amd.cda.kernels_cuda.fa2_cda import prefill_source
    monkeypatch.delenv("CDA_PREFILL_SOURCE", raising=False)
    assert prefill_source(3, H_KV, 300, 300) == "dense"
    sc = Scenario(gpu, seed=79, nmax=320)
    print("[backend] long prefill step lens=[300,5,260]", flush=True)
    out, cache, Q, cu = sc.step([300, 5, 260])
    check(out, sc.expected_prefill(cache, Q, cu, [0, 1, 2]))
    print("[backend] decode after the long prefill", flush=True)
    out, cache, Q, cu = sc.step([1, 1, 1])
    check(out, sc.expected_decode(cache, Q, cu, [0, 1, 2]))


@pytest.mark.parametrize("route", ["fa2_rawkv", "fa2_cda_rawkv", "fa2_cda_fused_rawkv"])
def test_backend_rawkv_routes(gpu, monkeypatch, route):
    """CDA_PREFILL_BACKEND raw-K/V routes (cda_attn_v2.py:1402-1441): a first
    prefill (no prefix: FA2 over the fresh K/V, unrotated for fa2_rawkv,
    rotated otherwise) then a chunked-prefill step
    (compressed prefix + fresh chunk: the hybrid kernel), each against the
    checker's hybrid_prefill on the cache the GPU wrote."""
    monkeypatch.setenv("CDA_PREFILL_BACKEND", route)
    sc = Scenario(gpu, seed=80)
    for lens in ([37, 100, 64], [20, 5, 33]):
        print(f"[backend] {route} step {lens}", flush=True)
        out, cache, Q, cu = sc.step(lens)
        K, V = sc.last_kv
        if route == "fa2_rawkv" and int(sc.lens.max()) == max(lens):
            from tests.cases import raw_causal_attention
            exp = raw_causal_attention(Q, np.asarray(cu, np.int32), K, V)
        else:
            exp = O.hybrid_prefill(Q, np.asarray(cu, np.int32), K, V, cache, sc.bt, sc.lens,
                                   sc.cb, sc.cb, O.hadamard128(), H_kv=H_KV, block_size=BS)
        check(out, exp)
