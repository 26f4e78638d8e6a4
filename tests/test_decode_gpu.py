"""GPU parity of the split-K decode against the CPU checker (through the C ABI).

Tolerance: 2e-3 max-abs on fp16 outputs against the fp32/fp64 checker run on
the same compressed cache."""
import json

import numpy as np
import pytest
import torch

from oracle import cda_oracle as O
from oracle import synth
from tests.cases import make_decode_case

pytestmark = pytest.mark.gpu
TOL = 2e-3


def run_gpu_decode(case, dev, *, gs, tile_n=0, max_seq_len=None, scale=None, cb_copy=False):
    from sub0_amd import _native
    q = torch.from_numpy(case.q.copy()).to(dev)
    cache = torch.from_numpy(case.cache).to(dev)
    bt = torch.from_numpy(case.block_table).to(dev)
    sl = torch.from_numpy(case.seq_lens).to(dev)
    cb = torch.from_numpy(case.cb_k).to(dev)
    cbv = cb if (case.cb_v is case.cb_k and not cb_copy) else torch.from_numpy(case.cb_v.copy()).to(dev)
    R = torch.from_numpy(case.R).to(dev)
    out = torch.full_like(q, float("nan"))
    msl = int(case.seq_lens.max()) if max_seq_len is None else max_seq_len
    _native.decode(q, cache, bt, sl, cb, cbv, R, R.half(), out, group_size=gs,
                   block_size=case.block_size, tile_n=tile_n, max_seq_len=msl,
                   scale=scale if scale is not None else 1.0 / np.sqrt(128))
    torch.cuda.synchronize()
    return out.cpu().numpy()


def check(out, exp, tol=TOL):
    assert np.isfinite(out).all(), "non-finite output"
    err = np.abs(out.astype(np.float32) - exp.astype(np.float32)).max()
    assert err <= tol, f"max abs err {err}"
    return err


CASES = [
    # (name, seq_lens, H_kv, gs, block_size, tile_n, fill)
    ("small_gqa", [300, 77], 2, 4, 16, 0, 0),
    ("cfg0_shape", [4096], 8, 4, 16, 0, 0),
    ("one_token", [1], 8, 4, 16, 0, 0xFF),
    ("ragged", [33, 1000, 17, 2049], 8, 4, 16, 0, 0xFF),
    ("gs8", [500, 1500], 8, 8, 16, 0, 0),
    ("block32", [999, 64], 8, 4, 32, 0, 0xFF),
    ("tile64", [2000], 8, 4, 16, 64, 0),
    ("tile_big", [1500], 8, 4, 16, 4096, 0),
    ("hkv4", [1234], 4, 4, 16, 0, 0),
    ("hkv9", [700, 31], 9, 4, 16, 0, 0xFF),
]


@pytest.mark.parametrize("name,seq_lens,H_kv,gs,bs,tile_n,fill", CASES, ids=[c[0] for c in CASES])
def test_decode_matches_checker(gpu, name, seq_lens, H_kv, gs, bs, tile_n, fill):
    print(f"[decode] case={name} seq_lens={seq_lens} H_kv={H_kv} gs={gs} bs={bs}", flush=True)
    case = make_decode_case(1000 + len(name), seq_lens, H_kv=H_kv, gs=gs, block_size=bs,
                            fill=fill)
    out = run_gpu_decode(case, gpu, gs=gs, tile_n=tile_n)
    check(out, case.expected)


@pytest.mark.parametrize("name,seq_lens,gs,bs,tile_n", [
    ("cfg0_shape", [4096], 4, 16, 0),
    ("ragged", [33, 1000, 17, 2049], 4, 16, 0),
    ("gs8", [500, 1500], 8, 16, 0),
    ("block32_tile64", [999, 64], 4, 32, 64),
])
def test_decode_general_kernel_matches_checker(gpu, name, seq_lens, gs, bs, tile_n):
    """The same 8-head, 144-byte-slot cases with the page-streaming kernel
    forbidden: the general kernel must meet the same bar, and both kernels
    must agree with each other."""
    from sub0_amd import _native
    print(f"[decode-general] case={name} seq_lens={seq_lens} gs={gs} bs={bs}", flush=True)
    case = make_decode_case(2000 + len(name), seq_lens, H_kv=8, gs=gs, block_size=bs, fill=0xFF)
    streamed = run_gpu_decode(case, gpu, gs=gs, tile_n=tile_n)
    _native.set_stream_kernel(False)
    try:
        general = run_gpu_decode(case, gpu, gs=gs, tile_n=tile_n)
    finally:
        _native.set_stream_kernel(True)
    check(general, case.expected)
    check(streamed, case.expected)
    check(streamed, general, tol=1e-3)


@pytest.mark.parametrize("seed,seq_lens", [(6, [65, 64, 63, 1]), (80, [1, 2, 3, 5, 9, 17])])
def test_decode_short_sequences(gpu, seed, seq_lens):
    """Few keys, so outputs reach |x| ~ 3 where one fp16 ulp is ~2e-3: V must
    be rebuilt as fp16(centroid * norm) per element, as the reference decodes
    it (a norm folded into P put these cases 2 ulps off).  Both kernels."""
    from sub0_amd import _native
    print(f"[decode-short] seed={seed} seq_lens={seq_lens}", flush=True)
    case = make_decode_case(seed, seq_lens, H_kv=8, gs=4, fill=0xFF)
    check(run_gpu_decode(case, gpu, gs=4), case.expected)
    _native.set_stream_kernel(False)
    try:
        check(run_gpu_decode(case, gpu, gs=4), case.expected)
    finally:
        _native.set_stream_kernel(True)


K2V2_CASES = [
    # name, seq_lens, gs, block_size, tile_n, fill
    ("k2v2_ragged", [300, 1, 77, 1031], 4, 16, 0, 0xFF),
    ("k2v2_gs8", [500, 1200], 8, 16, 0, 0),
    ("k2v2_tile64", [2000], 4, 16, 64, 0xFF),
    ("k2v2_short", [1, 2, 3, 5, 9, 17, 65], 4, 16, 0, 0xFF),
    ("k2v2_block32", [999, 64], 4, 32, 0, 0xFF),
]


@pytest.mark.parametrize("name,seq_lens,gs,bs,tile_n,fill", K2V2_CASES,
                         ids=[c[0] for c in K2V2_CASES])
def test_decode_k2v2_matches_checker(gpu, codebooks, name, seq_lens, gs, bs, tile_n, fill):
    """2-bit K and V codes (4-level codebook, 80-byte slots; pack_2bit,
    compression.py:375-397) through the page-streaming kernel (8 KV heads, one
    codebook) and the general kernel; both meet the bar and agree."""
    from sub0_amd import _native
    print(f"[decode-k2v2] case={name} seq_lens={seq_lens} gs={gs} bs={bs}", flush=True)
    cb4 = codebooks["lloyd_beta4"].astype(np.float32)
    case = make_decode_case(5000 + len(name), seq_lens, H_kv=8, gs=gs, block_size=bs, cb=cb4,
                            fill=fill)
    assert case.cache.shape[-1] == 80
    streamed = run_gpu_decode(case, gpu, gs=gs, tile_n=tile_n)
    check(streamed, case.expected)
    _native.set_stream_kernel(False)
    try:
        general = run_gpu_decode(case, gpu, gs=gs, tile_n=tile_n)
    finally:
        _native.set_stream_kernel(True)
    check(general, case.expected)
    check(streamed, general, tol=1e-3)


def test_decode_k2v2_separate_codebooks(gpu, codebooks):
    """K2V2 with different K and V codebooks (Lloyd and uniform)."""
    cbk = codebooks["lloyd_beta4"].astype(np.float32)
    cbv = codebooks["uniform4"].astype(np.float32)
    case = make_decode_case(5100, [640, 99], H_kv=8, gs=4, cb=cbk, cb_v=cbv, fill=0xFF)
    check(run_gpu_decode(case, gpu, gs=4), case.expected)


def test_decode_separate_equal_codebooks(gpu):
    """cb_K and cb_V as separate tensors with equal values (the reference
    passes one Compressor's codebook each)."""
    case = make_decode_case(3001, [700, 1300], H_kv=8, gs=4, fill=0xFF)
    out = run_gpu_decode(case, gpu, gs=4, cb_copy=True)
    check(out, case.expected)


def test_decode_different_v_codebook(gpu):
    """V encoded with its own codebook (uniform 16 levels): K and V tables differ."""
    cbv = O.uniform_centroids(16)
    case = make_decode_case(3002, [900, 33], H_kv=8, gs=4, cb_v=cbv, fill=0xFF)
    out = run_gpu_decode(case, gpu, gs=4)
    check(out, case.expected)


def test_decode_scale_and_slack_max_seq_len(gpu):
    """Non-default softmax scale; max_seq_len larger than every seq_len."""
    case = make_decode_case(77, [400, 250], H_kv=8, gs=4, scale=0.3)
    out = run_gpu_decode(case, gpu, gs=4, max_seq_len=1000, scale=0.3)
    check(out, case.expected)


@pytest.mark.parametrize("scale", [None, 0.5], ids=["default_scale", "scale0.5"])
def test_decode_rising_scores(gpu, scale):
    """K rows growing 6x along the sequence: the running max keeps moving, so
    the O rescale runs on many chunks (both split kernels)."""
    from sub0_amd import _native
    print(f"[decode] rising scores scale={scale}", flush=True)
    case = make_decode_case(3100 + (scale is not None), [4000, 1500, 37], H_kv=8, gs=4,
                            scale=scale, fill=0xFF, k_ramp=5.0)
    check(run_gpu_decode(case, gpu, gs=4, scale=scale), case.expected)
    _native.set_stream_kernel(False)
    try:
        check(run_gpu_decode(case, gpu, gs=4, scale=scale), case.expected)
    finally:
        _native.set_stream_kernel(True)


def test_decode_empty_sequence_gives_zero(gpu):
    case = make_decode_case(78, [0, 200], H_kv=8, gs=4)
    out = run_gpu_decode(case, gpu, gs=4, max_seq_len=200)
    assert np.all(out[0] == 0)
    check(out[1:], case.expected[1:])


def test_decode_golden_cfg0(gpu, golden, codebooks):
    """BASELINE config 0 on the reference's own encoded cache and output."""
    g = golden("attn_cfg0.npz")
    meta = json.loads((__import__("pathlib").Path(__file__).parent / "golden" /
                       "attn_cfg0.json").read_text())
    B, H_kv, N = meta["B"], meta["H_kv"], meta["N"]
    cb = codebooks["lloyd_beta16"]
    bt = synth.permuted_block_table(meta["seed"], B, N // 16)
    cache = O.build_paged_cache(g["k_idx"], g["k_norm"], g["v_idx"], g["v_norm"], bt, 16, 16)
    from tests.cases import DecodeCase
    R = codebooks["hadamard128"]
    exp = O.decode_paged(g["q"][:, :, 0], cache, bt, np.full(B, N, np.int32), cb, cb, R,
                         H_kv=H_kv, block_size=16)
    case = DecodeCase(g["q"][:, :, 0].copy(), cache, bt, np.full(B, N, np.int32), cb, cb, R,
                      H_kv, 16, exp)
    out = run_gpu_decode(case, gpu, gs=4)
    check(out, exp)
    check(out, g["out"][:, :, 0])


def test_decode_graph_replay(gpu):
    """Captured decode replays match eager output on every replay."""
    from sub0_amd.cda.kernels_cuda.wrappers import decode_hmma_v1
    case = make_decode_case(91, [777, 1500, 64], H_kv=8, gs=4)
    dev = gpu
    q = torch.from_numpy(case.q.copy()).to(dev)
    cache = torch.from_numpy(case.cache).to(dev)
    bt = torch.from_numpy(case.block_table).to(dev)
    sl = torch.from_numpy(case.seq_lens).to(dev)
    cb = torch.from_numpy(case.cb_k).to(dev)
    cbv = cb.clone()        # separate tensors with equal values, as the reference passes them
    R = torch.from_numpy(case.R).to(dev)
    out = torch.empty_like(q)

    def call():
        decode_hmma_v1(q, cache, bt, sl, out, cb_K=cb, cb_V=cbv, rotation_fp32=R,
                       rotation_fp16=R.half(), group_size=4, block_size=16, max_seq_len=1500)

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(3):
            call()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    eager = out.clone()
    check(eager.cpu().numpy(), case.expected)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        call()
    for _ in range(3):
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)


@pytest.mark.parametrize("same_values", [True, False], ids=["equal_cb", "different_cb"])
def test_decode_capture_first(gpu, same_values):
    """Graph capture before any eager call, with K and V codebooks passed as
    two tensors: the kernel choice is made on the device, so the replays are
    right for equal and for different codebooks."""
    from sub0_amd import _native
    print(f"[decode] capture first, same_values={same_values}", flush=True)
    cbv_np = None if same_values else O.uniform_centroids(16)
    case = make_decode_case(3100, [1100, 40, 2500], H_kv=8, gs=4, fill=0xFF, cb_v=cbv_np)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(gpu)
    q, cache, bt, sl = t(case.q), t(case.cache), t(case.block_table), t(case.seq_lens)
    cb = t(case.cb_k)
    cbv = t(case.cb_v.copy())                       # a distinct tensor in both cases
    R = t(case.R)
    out = torch.full_like(q, float("nan"))
    ws = torch.empty(_native.decode_workspace_size(3, 32, 8, 2500) + 256, dtype=torch.uint8,
                     device=gpu)

    def call():
        _native.decode(q, cache, bt, sl, cb, cbv, R, R.half(), out, group_size=4, block_size=16,
                       tile_n=0, max_seq_len=2500, scale=float(1 / np.sqrt(128)), workspace=ws)

    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            call()
    torch.cuda.current_stream().wait_stream(s)
    for _ in range(3):
        out.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        check(out.cpu().numpy(), case.expected)


def _plan_fused(B, n, cus=256):
    """Host restatement of the single-launch plan (splits per sequence), to
    label the cases below by the path they take."""
    n = max(n, 1)
    s = max(1, min(-(-cus // (8 * B)), -(-n // 512)))
    s = max(s, -(-n // 65536))
    wg = -(-(-(-n // s)) // 512) * 512
    return -(-n // wg)


FUSED_CASES = [
    # name, seq_lens, gs, levels, block_size
    ("b8_xcd_combine", [700, 64, 1, 4096, 300, 2049, 65, 1000], 4, 16, 16),
    ("b3_combine", [5000, 17, 900], 4, 16, 16),
    ("b1_long_combine", [20000], 4, 16, 16),
    ("b32_single_launch", [int(x) for x in np.random.default_rng(7).integers(1, 1600, 32)],
     4, 16, 16),
    ("b32_gs8_single_launch", [int(x) for x in np.random.default_rng(8).integers(1, 900, 32)],
     8, 16, 32),
    ("b5_empty_mixed", [0, 513, 0, 64, 1], 4, 16, 16),
    ("b32_k2v2_single_launch", [int(x) for x in np.random.default_rng(9).integers(1, 1300, 32)],
     4, 4, 16),
    ("b2_k2v2_gs8_combine", [3000, 777], 8, 4, 16),
    ("b3_block48_combine", [2500, 48, 1100], 4, 16, 48),
    ("b32_block64_single_launch", [int(x) for x in np.random.default_rng(10).integers(1, 1000, 32)],
     4, 16, 64),
]


@pytest.mark.parametrize("name,seq_lens,gs,levels,bs", FUSED_CASES,
                         ids=[c[0] for c in FUSED_CASES])
def test_decode_single_launch_matches_checker(gpu, codebooks, name, seq_lens, gs, levels, bs):
    """The single-launch decode (one workgroup per sequence x split x KV head:
    in-kernel q rotation, eight waves on consecutive token ranges merged in
    LDS, the R^T epilogue in the kernel when one split covers the sequence,
    the combine launch otherwise) against the checker, and against the
    three-launch form on the same inputs."""
    from sub0_amd import _native
    B, n = len(seq_lens), max(seq_lens)
    print(f"[decode-fused] case={name} B={B} max_n={n} gs={gs} levels={levels} bs={bs} "
          f"splits={_plan_fused(B, n)}", flush=True)
    cb = None if levels == 16 else codebooks["lloyd_beta4"].astype(np.float32)
    case = make_decode_case(7000 + len(name), seq_lens, H_kv=8, gs=gs, block_size=bs, cb=cb,
                            fill=0xFF)
    fused = run_gpu_decode(case, gpu, gs=gs)
    _native.set_fused_kernel(False)
    try:
        three = run_gpu_decode(case, gpu, gs=gs)
    finally:
        _native.set_fused_kernel(True)
    for b in range(B):
        if seq_lens[b] == 0:
            assert np.all(fused[b] == 0)
    check(fused, case.expected)
    check(three, case.expected)
    check(fused, three, tol=1e-3)


@pytest.mark.parametrize("seq_lens", [[1500] * 32, [9000, 3]], ids=["single", "combine"])
def test_decode_single_launch_graph_replay(gpu, seq_lens):
    """The single-launch decode captured in a graph: every replay equals the
    eager output."""
    case = make_decode_case(7100 + len(seq_lens), seq_lens, H_kv=8, gs=4, fill=0xFF)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(gpu)
    q, cache, bt, sl, cb, R = (t(case.q), t(case.cache), t(case.block_table),
                               t(case.seq_lens), t(case.cb_k), t(case.R))
    out = torch.full_like(q, float("nan"))
    from sub0_amd import _native

    def call():
        _native.decode(q, cache, bt, sl, cb, cb, R, R.half(), out, group_size=4, block_size=16,
                       tile_n=0, max_seq_len=max(seq_lens), scale=float(1 / np.sqrt(128)))

    call()
    torch.cuda.synchronize()
    eager = out.clone()
    check(eager.cpu().numpy(), case.expected)
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        call()
        with torch.cuda.graph(g, stream=s):
            call()
    torch.cuda.current_stream().wait_stream(s)
    for _ in range(3):
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)


def test_decode_single_launch_slack_max_seq_len(gpu):
    """max_seq_len far above every sequence (the plan covers tokens no
    sequence has): same result as the tight bound."""
    case = make_decode_case(7200, [900, 33, 2000], H_kv=8, gs=4, fill=0xFF)
    tight = run_gpu_decode(case, gpu, gs=4)
    slack = run_gpu_decode(case, gpu, gs=4, max_seq_len=60000)
    check(slack, case.expected)
    check(slack, tight, tol=1e-3)


def test_decode_single_launch_all_empty(gpu):
    """Every sequence empty and max_seq_len 0: the single launch writes zeros."""
    case = make_decode_case(7300, [0, 0, 0], H_kv=8, gs=4)
    out = run_gpu_decode(case, gpu, gs=4, max_seq_len=0)
    assert np.all(out == 0)


def test_decode_single_launch_two_rounds(gpu):
    """B=64: 512 single-split workgroups, two per CU over the run (the XCD
    mapping over 64 sequences)."""
    from sub0_amd import _native
    rng = np.random.default_rng(11)
    seq = [int(x) for x in rng.integers(1, 700, 64)]
    assert _native.decode_fused_plan(64, 8, max(seq))[1] == 1
    case = make_decode_case(7400, seq, H_kv=8, gs=4, fill=0xFF)
    check(run_gpu_decode(case, gpu, gs=4), case.expected)
