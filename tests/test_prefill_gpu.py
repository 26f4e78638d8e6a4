"""GPU parity of the causal varlen prefill (config 3) and its helpers against
the CPU checker (through the C ABI and the reference-shaped mirror).

Tolerances: attention outputs 2e-3 max-abs (fp16 outputs against the checker
on the same compressed cache); the dense rotated K/V are
bit-exact (fp16(centroid * norm)); the Hadamard helper is within one fp16
rounding of the exact transform."""
import numpy as np
import pytest
import torch

from oracle import cda_oracle as O
from oracle import synth
from tests.cases import make_prefill_case

pytestmark = pytest.mark.gpu
TOL = 2e-3


def _dev(x, dev):
    return torch.from_numpy(np.ascontiguousarray(x)).to(dev)


def run_prefill(case, dev, *, dense=False, scale=None, split=False, max_seq_len=None, pad_rows=0):
    from sub0_amd import _native
    q = _dev(case.q, dev)
    if pad_rows:
        q = torch.cat([q, torch.zeros((pad_rows,) + tuple(q.shape[1:]), dtype=q.dtype, device=dev)])
    out = torch.full_like(q, float("nan"))
    cache = _dev(case.cache, dev)
    bt = _dev(case.block_table, dev)
    cu = _dev(case.cu_q, dev)
    sk = _dev(case.seq_k, dev)
    cb = _dev(case.cb, dev)
    cbv = cb if case.cb_v is None else _dev(case.cb_v, dev)
    sc = scale if scale is not None else 1.0 / np.sqrt(128)
    max_q = int(np.diff(case.cu_q).max()) if len(case.cu_q) > 1 else 0
    max_k = int(case.seq_k.max())
    if dense:
        k_rot, v_rot = _native.paged_to_dense(cache, bt, sk, cb, cbv, block_size=case.block_size,
                                              max_seq_len=max_k)
        cu_k = torch.arange(0, len(case.seq_k) + 1, dtype=torch.int32, device=dev) * max_k
        _native.fa2_varlen_fwd_hadamard(q, k_rot, v_rot, out, cu, cu_k, sk, max_q, max_k, sc)
    else:
        _native.prefill_paged(q, cache, bt, cu, sk, cb, cbv, out, block_size=case.block_size,
                              max_query_len=max_q, scale=sc,
                              max_seq_len=(max_seq_len or max_k) if split else None)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def check(out, exp, tol=TOL):
    assert np.isfinite(out).all(), "non-finite output"
    err = float(np.abs(out.astype(np.float32) - exp.astype(np.float32)).max()) if out.size else 0.0
    assert err <= tol, f"max abs err {err}"
    return err


CASES = [
    # name, seq_q, seq_k, H_kv, gs
    ("one_seq_full", [300], [300], 8, 4),
    ("ragged_full", [17, 64, 129, 200], [17, 64, 129, 200], 8, 4),
    ("with_past", [40, 1, 96], [300, 77, 96], 8, 4),
    ("gs8", [150, 70], [150, 90], 4, 8),
    ("hkv2", [513], [513], 2, 4),
    ("one_token", [1, 1], [1, 33], 8, 4),
]


@pytest.mark.parametrize("name,seq_q,seq_k,H_kv,gs", CASES, ids=[c[0] for c in CASES])
@pytest.mark.parametrize("dense", [False, True], ids=["paged", "dense"])
def test_prefill_matches_checker(gpu, name, seq_q, seq_k, H_kv, gs, dense):
    print(f"[prefill] case={name} dense={dense} seq_q={seq_q} seq_k={seq_k}", flush=True)
    case = make_prefill_case(4000 + len(name), seq_q, seq_k, H_kv=H_kv, gs=gs, fill=0xFF)
    out = run_prefill(case, gpu, dense=dense)
    check(out, case.expected)


@pytest.mark.parametrize("mode", ["paged", "dense", "key_split"])
def test_prefill_rising_scores(gpu, mode):
    """K rows growing 11x along each sequence: the lazy running max moves
    past its first tile (about twice per query row on average).  (At a
    softmax scale several times the default, scores this large turn the
    last-bit rounding of q_rot -- the Hadamard MFMA's order, as the
    reference's own hadamard128 helper, not the checker's sequential fp32
    sum -- into errors above 2e-3, as they would for the reference.)"""
    print(f"[prefill] rising scores mode={mode}", flush=True)
    case = make_prefill_case(4650, [700, 96, 16], [700, 1400, 3000], H_kv=8, gs=4, k_ramp=10.0)
    check(run_prefill(case, gpu, dense=(mode == "dense"), split=(mode == "key_split")),
          case.expected)


@pytest.mark.parametrize("split", [False, True], ids=["unsplit", "key_split"])
@pytest.mark.parametrize("copy", [False, True], ids=["different", "equal_copy"])
def test_prefill_separate_codebooks(gpu, split, copy):
    """V encoded with its own codebook (uniform 16 levels), or a separate
    tensor with the K codebook's values: the compressed-tile kernel builds one
    shared table or two half tables."""
    print(f"[prefill] separate codebooks split={split} copy={copy}", flush=True)
    cbv = synth_cb_copy() if copy else O.uniform_centroids(16)
    case = make_prefill_case(4600 + 2 * split + copy, [16, 150] if split else [130, 64],
                             [3000, 1700] if split else [300, 64], H_kv=8, gs=4, fill=0xFF,
                             cb_v=cbv)
    check(run_prefill(case, gpu, split=split), case.expected)
    check(run_prefill(case, gpu, dense=True), case.expected)


def synth_cb_copy():
    from tests.cases import synth_cb
    return synth_cb().copy()


@pytest.mark.parametrize("dense", [False, True], ids=["paged", "dense"])
def test_prefill_negative_scale(gpu, dense):
    """A negative softmax scale (folded into the sign of q_rot in the kernel)."""
    print(f"[prefill] negative scale dense={dense}", flush=True)
    case = make_prefill_case(4500, [90, 33], [120, 33], H_kv=8, gs=4, scale=-0.15)
    out = run_prefill(case, gpu, dense=dense, scale=-0.15)
    check(out, case.expected)


@pytest.mark.parametrize("block_size", [32, 48])
def test_prefill_larger_blocks(gpu, block_size):
    """Pages of 32 and 48 tokens (the block-table entries are fetched one tile
    ahead; 48 is not a power of two)."""
    print(f"[prefill] block_size={block_size}", flush=True)
    case = make_prefill_case(4400 + block_size, [200, 97], [260, 97], H_kv=8, gs=4,
                             block_size=block_size, fill=0xFF)
    out = run_prefill(case, gpu, dense=False)
    check(out, case.expected)


def test_prefill_scale_and_empty_sequence(gpu):
    """Non-default scale; a sequence with no queries between two others."""
    case = make_prefill_case(4100, [33, 0, 70], [33, 50, 100], H_kv=8, gs=4, scale=0.2)
    out = run_prefill(case, gpu, scale=0.2)
    check(out, case.expected)


def test_prefill_golden_causal(gpu, golden, codebooks):
    """The reference's own causal output (B=1, 8 Q / 2 KV heads, 37 queries
    over 200 keys) on the reference-encoded cache."""
    from sub0_amd import _native
    a = golden("attn_causal.npz")
    cb = codebooks["lloyd_beta16"]
    meta = a["meta"]
    B, H_q, H_kv, N, M = (int(x) for x in meta[:5])
    bt = synth.permuted_block_table(9, B, (N + 15) // 16)
    cache = O.build_paged_cache(a["k_idx"], a["k_norm"], a["v_idx"], a["v_norm"], bt, 16, 16)
    q = a["q"][0].transpose(1, 0, 2).copy()
    dev = gpu
    qd = _dev(q, dev)
    out = torch.empty_like(qd)
    _native.prefill_paged(qd, _dev(cache, dev), _dev(bt, dev),
                          torch.tensor([0, M], dtype=torch.int32, device=dev),
                          torch.tensor([N], dtype=torch.int32, device=dev), _dev(cb, dev),
                          _dev(cb, dev), out, block_size=16, max_query_len=M,
                          scale=1.0 / np.sqrt(128))
    ref = a["out"][0].transpose(1, 0, 2)
    check(out.cpu().numpy(), ref)


def test_dense_loader_bit_exact(gpu):
    """paged -> dense rotated K/V: fp16(centroid * norm) rows, zeros past seq_lens."""
    from sub0_amd import _native
    case = make_prefill_case(4200, [5, 5], [77, 20], H_kv=8, gs=4, fill=0xFF)
    dev = gpu
    max_k = 80
    k_rot, v_rot = _native.paged_to_dense(_dev(case.cache, dev), _dev(case.block_table, dev),
                                          _dev(case.seq_k, dev), _dev(case.cb, dev),
                                          _dev(case.cb, dev), block_size=16, max_seq_len=max_k)
    k_rot = k_rot.cpu().numpy().reshape(2, max_k, 8, 128)
    v_rot = v_rot.cpu().numpy().reshape(2, max_k, 8, 128)
    for b in range(2):
        n = int(case.seq_k[b])
        t = np.arange(n)
        slots = case.block_table[b, t // 16] * 16 + t % 16
        rows = case.cache[slots]                                   # (n, 8, 144)
        for tensor, code0, norm0 in ((k_rot, 0, 128), (v_rot, 64, 132)):
            idx = O.unpack_4bit(rows[:, :, code0:code0 + 64])
            norm = rows[:, :, norm0:norm0 + 4].copy().view(np.float32)[..., 0]
            exp = (case.cb[idx] * norm[..., None]).astype(np.float16)
            assert np.array_equal(tensor[b, :n].view(np.uint16), exp.view(np.uint16))
            assert not tensor[b, n:].any()


def test_hadamard128_helper(gpu):
    from sub0_amd import _native
    rng = np.random.default_rng(5)
    x = rng.standard_normal((1000, 128)).astype(np.float16)
    xd = _dev(x, gpu)
    y = torch.empty_like(xd)
    _native.hadamard128(xd, y, 1.0 / np.sqrt(128))
    exact = x.astype(np.float64) @ O.hadamard128().astype(np.float64)
    got = y.cpu().numpy().astype(np.float64)
    ulp = np.spacing(np.abs(exact).astype(np.float16)).astype(np.float64)
    assert (np.abs(got - exact) <= ulp).all()


def test_dropin_prefill_wrapper(gpu):
    """fa2_cda_prefill_varlen_v1 through the reference-shaped mirror, fused
    (compressed tiles) and with return_dense_kv (dense bridge)."""
    from sub0_amd.cda.kernels_cuda.fa2_cda import fa2_cda_prefill_varlen_v1
    case = make_prefill_case(4300, [100, 31], [130, 31], H_kv=8, gs=4)
    dev = gpu
    R = _dev(O.hadamard128(), dev)
    args = (_dev(case.q, dev), _dev(case.cache, dev), _dev(case.block_table, dev),
            _dev(case.cu_q, dev), _dev(case.seq_k, dev))
    for dense in (False, True):
        out = torch.empty_like(args[0])
        r = fa2_cda_prefill_varlen_v1(*args, out, cb_K=_dev(case.cb, dev), cb_V=_dev(case.cb, dev),
                                      rotation_fp32=R, group_size=4, block_size=16,
                                      max_query_len=100, max_seq_len=130,
                                      fuse_fa2_epilogue=True, return_dense_kv=dense)
        torch.cuda.synchronize()
        check(out.cpu().numpy(), case.expected)
        assert (r is not None) == dense


# Key-split prefill (cda_prefill_paged_hadamard_ws): short query chunks over long
# contexts; ragged key lengths leave some splits without keys.
SPLIT_CASES = [
    # name, seq_q, seq_k, H_kv, gs
    ("short_chunk", [16], [4000], 8, 4),
    ("ragged", [5, 30, 1], [700, 2000, 1500], 8, 4),
    ("gs8", [20], [3000], 4, 8),
    ("one_token", [1, 1], [1, 1200], 8, 4),
    ("chunk_not_multiple", [40], [2333], 8, 4),
]


@pytest.mark.parametrize("name,seq_q,seq_k,H_kv,gs", SPLIT_CASES, ids=[c[0] for c in SPLIT_CASES])
def test_prefill_key_split_matches_checker(gpu, name, seq_q, seq_k, H_kv, gs):
    from sub0_amd import _native
    print(f"[prefill-split] case={name} seq_q={seq_q} seq_k={seq_k}", flush=True)
    case = make_prefill_case(4700 + len(name), seq_q, seq_k, H_kv=H_kv, gs=gs, fill=0xFF)
    T = int(case.cu_q[-1])
    need = _native.prefill_workspace_size(len(seq_q), T, H_kv * gs, H_kv, max(seq_q), max(seq_k))
    assert need > 0, "the case is meant to take the key-split path"
    out = run_prefill(case, gpu, split=True)
    check(out, case.expected)
    ref = run_prefill(case, gpu)           # unsplit kernel on the same cache
    assert float(np.abs(out.astype(np.float32) - ref.astype(np.float32)).max()) <= 1e-3


def test_prefill_key_split_negative_scale(gpu):
    print("[prefill-split] negative scale", flush=True)
    case = make_prefill_case(4800, [12], [2500], H_kv=8, gs=4, scale=-0.15)
    out = run_prefill(case, gpu, scale=-0.15, split=True)
    check(out, case.expected)


@pytest.mark.parametrize("bound", ["larger", "smaller"])
def test_prefill_key_split_max_seq_len_bound(gpu, bound):
    """The split plan follows max_seq_len: a bound above every key length only
    adds empty splits, one below some length still covers every key (the last
    split runs to the end of the sequence)."""
    from sub0_amd import _native
    print(f"[prefill-split] max_seq_len {bound}", flush=True)
    case = make_prefill_case(4900, [16, 9], [3000, 1800], H_kv=8, gs=4)
    msl = 5000 if bound == "larger" else 1200
    T = int(case.cu_q[-1])
    assert _native.prefill_workspace_size(2, T, 32, 8, 16, msl) > 0
    out = run_prefill(case, gpu, split=True, max_seq_len=msl)
    check(out, case.expected)


def test_prefill_key_split_padded_query_rows(gpu):
    """q padded with rows past cu_seqlens_q[B]: the split path merges only the
    real rows and leaves the padding rows of out untouched (NaN here)."""
    print("[prefill-split] padded q rows", flush=True)
    case = make_prefill_case(4950, [12], [2500], H_kv=8, gs=4)
    out = run_prefill(case, gpu, split=True, pad_rows=5)
    check(out[:12], case.expected)
    assert np.isnan(out[12:]).all()
