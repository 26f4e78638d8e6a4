"""The C ABI library (CPU-side checks: loads, exports every declared symbol,
validates arguments before touching a device)."""
import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


def declared_symbols():
    text = (ROOT / "include" / "cda_hip.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(cda_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    from sub0_amd import _native
    L = _native.lib()
    syms = declared_symbols()
    assert len(syms) >= 7
    for s in syms:
        assert hasattr(L, s), s
    assert sorted(_native.SYMBOLS) == syms


def test_version_and_plan():
    from sub0_amd import _native
    assert _native.lib().cda_hip_version() >= 100
    tile, splits = _native.decode_plan(32, 32, 8, 65536)
    assert tile % 32 == 0 and tile * splits >= 65536 and splits <= 512
    tile, splits = _native.decode_plan(1, 32, 8, 4096, 100)
    assert tile == 128 and splits == 32
    assert _native.decode_plan(1, 32, 8, 0) == (32, 1)
    ws1 = _native.decode_workspace_size(4, 32, 8, 4096)
    ws2 = _native.decode_workspace_size(4, 32, 8, 65536)
    assert 0 < ws1 <= ws2 and ws1 % 256 == 0


def test_decode_fused_plan_fits_the_workspace():
    """The single-launch plan (256 CUs without a device): whole 64-token
    chunks per wave, at most 4096 pages per workgroup, every token covered,
    and never more splits than the three-launch plan, whose
    cda_decode_workspace_size() callers allocate."""
    from sub0_amd import _native
    assert _native.decode_fused_plan(32, 8, 65536) == (8192, 1)     # one launch per step
    assert _native.decode_fused_plan(32, 8, 4096) == (512, 1)
    assert _native.decode_fused_plan(1, 8, 4096) == (64, 8)         # one chunk per wave
    assert _native.decode_fused_plan(1, 8, 65536) == (256, 32)
    assert _native.decode_fused_plan(4, 8, 65536) == (1024, 8)
    assert _native.decode_fused_plan(32, 8, 262144) == (8192, 4)    # page-row table cap
    assert _native.decode_fused_plan(3, 8, 0) == (64, 1)
    for B in (1, 2, 3, 4, 5, 7, 8, 16, 31, 32, 64, 256):
        for n in (1, 63, 64, 65, 511, 512, 513, 1000, 4096, 16383, 16384, 65535, 65536,
                  65537, 131072, 262144, 1000003):
            wt, ns = _native.decode_fused_plan(B, 8, n)
            assert wt % 64 == 0 and 64 <= 8 * wt <= 65536, (B, n, wt)
            assert 8 * wt * ns >= n and 8 * wt * (ns - 1) < n, (B, n, wt, ns)
            _, ns3 = _native.decode_plan(B, 8 * 4, 8, n)
            assert ns <= ns3, (B, n, ns, ns3)
    with pytest.raises(ValueError):
        _native.decode_fused_plan(0, 8, 100)


def test_prefill_key_split_plan():
    """Host-side plan of the key-split prefill: split only short chunks over
    long contexts (grid under 256 workgroups, >= 4 key tiles per split, <= 64
    splits); the workspace holds (O, m, l) per split, query row and q-head."""
    from sub0_amd import _native
    ws = _native.prefill_workspace_size
    # 16 queries over 16K keys, 8 KV heads: 8 workgroups -> 32 splits of 8 tiles.
    assert ws(1, 16, 32, 8, 16, 16384) == 32 * 16 * 32 * 128 * 4 + 32 * 16 * 32 * 2 * 4
    # 1 query over 64K keys, 1 KV head: 1 workgroup -> min(256, 1024 // 4) -> 64 (the cap).
    assert ws(1, 1, 4, 1, 1, 65536) == 64 * 1 * 4 * 128 * 4 + 64 * 1 * 4 * 2 * 4
    # 4000 keys = 63 tiles: min(64, 63 // 4) = 15 splits -> 5 tiles each -> 13 splits.
    assert ws(1, 16, 32, 8, 16, 4000) == 13 * 16 * 32 * 128 * 4 + 13 * 16 * 32 * 2 * 4
    assert ws(1, 16, 32, 8, 16, 200) == 0            # too few keys to split
    assert ws(8, 8 * 4096, 32, 8, 4096, 8192) == 0   # config-3-sized grid fills the chip
    assert ws(0, 0, 32, 8, 16, 16384) == 0
    assert ws(1, 16, 32, 5, 16, 16384) == 0          # group size not 4 or 8


def test_invalid_arguments_are_rejected_before_launch():
    from sub0_amd import _native
    L = _native.lib()
    P = ctypes.c_void_p
    dummy = P(256)
    rc = L.cda_decode_full_hmma_v3(dummy, dummy, 16, 144, 8, dummy, 1, dummy, dummy, dummy, 16,
                                   dummy, None, dummy, 1, 32, 3, 16, 0, 16, 0.1, dummy, 1 << 20,
                                   None)
    assert rc == -1 and b"group_size" in L.cda_hip_last_error()
    rc = L.cda_decode_full_hmma_v3(dummy, dummy, 16, 144, 8, dummy, 1, dummy, dummy, dummy, 16,
                                   dummy, None, dummy, 1, 32, 4, 8, 0, 16, 0.1, dummy, 1 << 20,
                                   None)
    assert rc == -1 and b"block_size" in L.cda_hip_last_error()
    rc = L.cda_decode_full_hmma_v3(dummy, dummy, 16, 144, 8, dummy, 1, dummy, dummy, dummy, 16,
                                   dummy, None, dummy, 1, 32, 4, 16, 0, 16, 0.1, P(512), 16, None)
    assert rc == -3
    rc = L.cda_paged_encode_fused(dummy, dummy, 1024, 1024, dummy, 4, dummy, 16, 144, 8, dummy,
                                  dummy, 5, None)
    assert rc == -1 and b"levels" in L.cda_hip_last_error()
    rc = L.cda_paged_encode_fused(dummy, dummy, 1024, 1024, dummy, 4, dummy, 16, 72, 8, dummy,
                                  dummy, 16, None)
    assert rc == -1 and b"slot_bytes" in L.cda_hip_last_error()
    assert L.cda_paged_encode_fused(None, None, 0, 0, None, 0, None, 0, 0, 0, None, None, 16,
                                    None) == 0          # zero tokens: nothing to do
    assert L.cda_decode_set_timing_events(dummy, None) == -1


def test_prefill_arguments_are_rejected_before_launch():
    from sub0_amd import _native
    L = _native.lib()
    P = ctypes.c_void_p
    d = P(256)

    def call(slot_bytes, block_size, cache=d):
        return L.cda_prefill_paged_hadamard(d, cache, 64, slot_bytes, 8, d, 4, d, d, 1, d, d, 16,
                                            d, 8, 32, block_size, 8, 0.1, None)
    assert call(144, 24) == -1 and b"multiple of 16" in L.cda_hip_last_error()
    assert call(128, 16) == -1 and b"slot" in L.cda_hip_last_error()
    assert call(144, 16, P(260)) == -1 and b"aligned" in L.cda_hip_last_error()


def test_python_binding_refuses_cpu_tensors():
    import torch
    from sub0_amd import _native
    x = torch.zeros(4, 8, 128, dtype=torch.float16)
    with pytest.raises(ValueError, match="GPU"):
        _native.paged_encode(x, x, torch.zeros(4, dtype=torch.int32),
                             torch.zeros(4, 8, 144, dtype=torch.uint8),
                             torch.zeros(16), torch.zeros(16))
