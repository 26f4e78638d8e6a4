"""GPU parity of the class-(a) decode comparators (cda_attn_v2.py:1062-1250):
R2 (dense dequantised K/V, then attention) and R1 (compressed tiles
dequantised on chip) against the CPU checker's decode on the same cache, to
2e-3 max-abs, and through the backend's CDA_DECODE_BACKEND routes."""
import numpy as np
import pytest
import torch

from tests.cases import make_decode_case

pytestmark = pytest.mark.gpu
TOL = 2e-3


def _check(out, exp):
    assert np.isfinite(out).all()
    err = float(np.abs(out.astype(np.float32) - exp.astype(np.float32)).max())
    assert err <= TOL, f"max abs err {err}"


@pytest.mark.parametrize("route", ["dequant_fa2", "fused_dequant_fa2"])
@pytest.mark.parametrize("gs,seq_lens", [(4, [300, 1, 77, 1031]), (8, [500, 1200]),
                                         (4, [0, 65, 16])])
def test_comparator_matches_checker(gpu, route, gs, seq_lens):
    from sub0_amd.cda.kernels_cuda import class_a
    print(f"[class-a] route={route} gs={gs} seq_lens={seq_lens}", flush=True)
    case = make_decode_case(7000 + gs, seq_lens, H_kv=8, gs=gs, fill=0xFF)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(gpu)
    q, cache, bt, sl = t(case.q), t(case.cache), t(case.block_table), t(case.seq_lens)
    cb, R = t(case.cb_k), t(case.R)
    out = torch.full_like(q, float("nan"))
    scale = 1.0 / np.sqrt(128)
    if route == "dequant_fa2":
        class_a.dequant_fa2_decode(q, cache, bt, sl, out, cb_K=cb, cb_V=cb, rotation_fp32=R,
                                   block_size=case.block_size,
                                   max_seq_len=max(1, int(max(seq_lens))), scale=scale)
    else:
        class_a.fused_dequant_fa2_decode(q, cache, bt, sl, out, cb_K=cb, cb_V=cb,
                                         block_size=case.block_size, scale=scale)
    torch.cuda.synchronize()
    _check(out.cpu().numpy(), case.expected)


@pytest.mark.parametrize("route", ["dequant_fa2", "fused_dequant_fa2"])
def test_backend_decode_routes(gpu, monkeypatch, route):
    from sub0_amd.cda.kernels_cuda.vllm_integration import cda_attn_v2 as A
    from tests.test_backend_gpu import Scenario, check
    print(f"[class-a] backend route={route}", flush=True)
    sc = Scenario(gpu, seed=81)
    sc.step([90, 33, 150])
    monkeypatch.setattr(A, "_DECODE_BACKEND", route)
    out, cache, Q, cu = sc.step([1, 1, 1])
    check(out, sc.expected_decode(cache, Q, cu, [0, 1, 2]))
