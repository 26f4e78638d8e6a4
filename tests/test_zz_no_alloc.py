"""The allocation-free decode entry point (cda_decode_full_hmma_v3_noalloc):
same output as cda_decode_full_hmma_v3 with a caller workspace, on two calls
in a row (the second smaller, so stale scratch contents from the first would
show), called through the C ABI."""
import ctypes

import numpy as np
import pytest
import torch

from tests.cases import make_decode_case

pytestmark = pytest.mark.gpu


def _call_noalloc(case, dev, gs):
    from sub0_amd import _native
    q = torch.from_numpy(case.q.copy()).to(dev)
    cache = torch.from_numpy(case.cache).to(dev)
    bt = torch.from_numpy(case.block_table).to(dev)
    sl = torch.from_numpy(case.seq_lens).to(dev)
    cb = torch.from_numpy(case.cb_k).to(dev)
    R = torch.from_numpy(case.R).to(dev)
    out = torch.full_like(q, float("nan"))
    B, H_q, _ = q.shape
    num_slots, H_kv, slot_bytes = cache.shape
    P = ctypes.c_void_p
    rc = _native.lib().cda_decode_full_hmma_v3_noalloc(
        P(q.data_ptr()), P(cache.data_ptr()), num_slots, slot_bytes, H_kv,
        P(bt.data_ptr()), bt.stride(0), P(sl.data_ptr()), P(cb.data_ptr()), P(cb.data_ptr()),
        cb.numel(), P(R.data_ptr()), None, P(out.data_ptr()), B, H_q, gs, case.block_size, 0,
        int(case.seq_lens.max()), float(1.0 / np.sqrt(128)),
        P(torch.cuda.current_stream(dev).cuda_stream))
    assert rc == 0, _native.lib().cda_hip_last_error()
    torch.cuda.synchronize()
    return out.cpu().numpy()


def _call_with_workspace(case, dev, gs):
    from tests.test_decode_gpu import run_gpu_decode
    return run_gpu_decode(case, dev, gs=gs)


def test_noalloc_decode_matches_workspace_entry_point(gpu):
    cases = [
        ("large", [3000, 4096, 129], 8, 4),     # first call: more splits x sequences
        ("small", [700], 8, 4),                 # second call: fewer, on stale scratch
    ]
    for name, seq_lens, H_kv, gs in cases:
        print(f"[noalloc] case={name} seq_lens={seq_lens}", flush=True)
        case = make_decode_case(4100 + len(name), seq_lens, H_kv=H_kv, gs=gs, fill=0xFF)
        got = _call_noalloc(case, gpu, gs)
        ref = _call_with_workspace(case, gpu, gs)
        assert np.isfinite(got).all()
        assert np.array_equal(got.view(np.uint16), ref.view(np.uint16))
        assert np.abs(got.astype(np.float32) - case.expected.astype(np.float32)).max() <= 2e-3


def test_noalloc_decode_rejects_oversized_shape(gpu):
    from sub0_amd import _native
    L = _native.lib()
    limit = L.cda_decode_noalloc_max_workspace()
    assert limit == 16 << 20
    B, H_q, H_kv, N = 4096, 32, 8, 65536       # needs far more than 16 MiB of partials
    need = L.cda_decode_workspace_size(B, H_q, H_kv, N, 64)
    assert need > limit
    P = ctypes.c_void_p
    dummy = P(16)
    rc = L.cda_decode_full_hmma_v3_noalloc(
        dummy, dummy, 1, 144, H_kv, dummy, 1, dummy, dummy, dummy, 16, dummy, None, dummy,
        B, H_q, 4, 16, 64, N, 0.088, None)
    assert rc == -3                              # CDA_E_WORKSPACE, nothing launched
    assert b"16777216" in L.cda_hip_last_error()
