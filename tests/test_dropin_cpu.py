"""The drop-in Python surface (cda._prebuilt_loader, cda.kernels_cuda.*),
host-side behaviour only."""
import pytest
import torch


def test_alias_makes_reference_imports_work():
    import sub0_amd
    sub0_amd.install_cda_alias()
    import cda._prebuilt_loader as pl                      # noqa: F401
    from cda.kernels_cuda.wrappers import decode_hmma_v1, paged_encode_fused_cuda  # noqa: F401
    from cda.kernels_cuda.hmma_loader import load_decode_hmma
    assert callable(load_decode_hmma)
    from cda.algorithm.compression import Compressor
    assert Compressor(128).codebook.numel() == 16


def test_loader_names_and_errors():
    from sub0_amd.cda._prebuilt_loader import PrebuiltMissing, load_pybind_module
    from sub0_amd.cda.kernels_cuda import hmma_loader as H
    m = load_pybind_module("_v1_decode_hmma_k4v4_gs4")
    assert callable(m.cda_decode_full_hmma_v3)
    assert load_pybind_module("_v1_decode_hmma_k4v4_gs4") is m        # cached
    assert callable(H.load_paged_encode_fused().cda_paged_encode_fused)
    assert H.load_decode_hmma(group_size=8) is load_pybind_module("_v1_decode_hmma_k4v4_gs8")
    with pytest.raises(ValueError):
        H.load_decode_hmma(group_size=2)
    assert callable(H.load_kv_cache_update(k4v2=True).cda_paged_encode_fused)
    assert callable(H.load_decode_hmma(k4v2=True, group_size=4).cda_decode_full_hmma_v3)
    assert callable(H.load_fa2_cda_loader(k4v2=True).cda_fa2_paged_cache_to_dense_rotated)
    with pytest.raises(PrebuiltMissing):
        load_pybind_module("no_such_kernel")
    assert issubclass(PrebuiltMissing, ImportError)


def test_wrapper_type_checks_match_reference():
    from sub0_amd.cda.kernels_cuda.wrappers import paged_encode_fused_cuda, decode_hmma_v1
    k = torch.zeros(2, 8, 128)
    with pytest.raises(TypeError):
        paged_encode_fused_cuda(k, k, torch.zeros(2, dtype=torch.int32),
                                torch.zeros(4, 8, 144, dtype=torch.uint8),
                                cb_K=torch.zeros(16), cb_V=torch.zeros(16))
    k16 = torch.zeros(2, 8, 64, dtype=torch.float16)
    with pytest.raises(ValueError):
        paged_encode_fused_cuda(k16, k16, torch.zeros(2, dtype=torch.int32),
                                torch.zeros(4, 8, 144, dtype=torch.uint8),
                                cb_K=torch.zeros(16), cb_V=torch.zeros(16))
    q = torch.zeros(1, 32, 128, dtype=torch.float16)
    with pytest.raises(ValueError, match="fp16 output"):
        decode_hmma_v1(q, torch.zeros(16, 8, 144, dtype=torch.uint8),
                       torch.zeros(1, 1, dtype=torch.int32), torch.ones(1, dtype=torch.int32),
                       torch.zeros(1, 32, 128), cb_K=torch.zeros(16), cb_V=torch.zeros(16),
                       rotation_fp32=torch.eye(128), rotation_fp16=torch.eye(128).half(),
                       group_size=4, block_size=16, max_seq_len=1)


def test_choose_tile_n_policy():
    from sub0_amd.cda.kernels_cuda.wrappers import _choose_tile_n
    for B, N in ((1, 4096), (4, 65536), (32, 65536), (32, 1)):
        t = _choose_tile_n(N, B=B, H_q=32)
        assert t % 32 == 0 and t >= 32 and -(-N // t) <= 512


def test_prefill_source_policy(monkeypatch):
    """The prefill K/V source: the dense bridge for long query chunks whose
    dense K/V fit in 4 GiB, compressed tiles otherwise; the environment
    variable forces either and rejects other values."""
    from sub0_amd.cda.kernels_cuda.fa2_cda import prefill_source
    monkeypatch.delenv("CDA_PREFILL_SOURCE", raising=False)
    assert prefill_source(8, 8, 7643, 7643) == "dense"
    assert prefill_source(8, 8, 255, 7643) == "compressed"
    assert prefill_source(32, 8, 64, 4096) == "compressed"
    # 64 sequences x 65536 keys x 8 heads of fp16 K and V = 16 GiB: too large
    assert prefill_source(64, 8, 4096, 65536) == "compressed"
    monkeypatch.setenv("CDA_PREFILL_SOURCE", "compressed")
    assert prefill_source(8, 8, 7643, 7643) == "compressed"
    monkeypatch.setenv("CDA_PREFILL_SOURCE", "dense")
    assert prefill_source(32, 8, 64, 4096) == "dense"
    monkeypatch.setenv("CDA_PREFILL_SOURCE", "fast")
    with pytest.raises(ValueError):
        prefill_source(8, 8, 7643, 7643)


def test_torch_ops_schemas_and_fake_kernels():
    """Both torch.ops namespaces are registered with in-place annotations on
    the outputs, load_torch_ops_library returns them, and the fake kernels
    trace without a GPU."""
    from sub0_amd.cda._prebuilt_loader import PrebuiltMissing, load_torch_ops_library
    ns = load_torch_ops_library("cda_hip")
    assert ns is torch.ops.cda_hip
    sch = str(torch.ops.cda_hip.decode.default._schema)
    assert "Tensor(a!) out" in sch and "int group_size" in sch and sch.endswith("-> ()")
    assert "Tensor(a!) flat_cache" in str(torch.ops.cda_hip.encode.default._schema)
    assert "Tensor(a!) out" in str(torch.ops.cda_hip.prefill.default._schema)
    assert "Tensor(a!) y" in str(torch.ops.cda_hip.hadamard128.default._schema)
    fork = load_torch_ops_library("_cda_vllm_fa2_fork_C")
    for op in ("dequantize_compressed_kv", "varlen_fwd", "varlen_fwd_compressed_kv",
               "varlen_fwd_compressed_kv_fused"):
        assert hasattr(fork, op)
    fsch = str(fork.varlen_fwd_compressed_kv_fused.default._schema)
    # the reference's positional order (interface.py:434-461)
    names = [a.name for a in fork.varlen_fwd_compressed_kv_fused.default._schema.arguments]
    assert names[:13] == ["q", "k_idx", "k_norm", "v_idx", "v_norm", "cb_k", "cb_v", "out",
                          "cu_seqlens_q", "cu_seqlens_k", "seqused_k", "block_table",
                          "alibi_slopes"]
    assert names[-2:] == ["uniform_codebook", "gen"] and "Tensor[]" in fsch
    with pytest.raises(PrebuiltMissing):
        load_torch_ops_library("no_such_namespace")
    from torch._subclasses.fake_tensor import FakeTensorMode
    with FakeTensorMode():
        kv = torch.empty(64, 8, 144, dtype=torch.uint8, device="cuda")
        bt = torch.empty(2, 4, dtype=torch.int32, device="cuda")
        sl = torch.empty(2, dtype=torch.int32, device="cuda")
        cb = torch.empty(16, device="cuda")
        k, v = torch.ops.cda_hip.paged_to_dense(kv, bt, sl, cb, cb, 16, 40)
        assert k.shape == (80, 8, 128) and k.dtype == torch.float16
        ki = torch.empty(100, 8, 64, dtype=torch.uint8, device="cuda")
        kn = torch.empty(100, 8, device="cuda")
        kd, vd = fork.dequantize_compressed_kv(ki, kn, ki, kn, cb, cb)
        assert kd.shape == (100, 8, 128)


def test_fa2_fork_build_stub():
    from sub0_amd.cda.kernels_vllm_fa2_fork import build
    build.load()
    assert hasattr(torch.ops._cda_vllm_fa2_fork_C, "varlen_fwd")


def test_fa2_fork_varlen_returns_lse_shape_on_meta():
    """The fork's varlen op returns (out, softmax_lse) with softmax_lse in
    FlashAttention-2's varlen layout (H_q, total_q) fp32 (reference
    interface.py:234-258); the meta kernel gives the shapes without a GPU."""
    from sub0_amd.cda._prebuilt_loader import load_torch_ops_library
    fork = load_torch_ops_library("_cda_vllm_fa2_fork_C")
    q = torch.empty(6, 8, 128, dtype=torch.float16, device="meta")
    k = torch.empty(6, 2, 128, dtype=torch.float16, device="meta")
    cu = torch.empty(3, dtype=torch.int32, device="meta")
    out, lse = fork.varlen_fwd(q, k, k, None, cu, cu, None, None, None, None, 4, 4, 0.0, 0.1,
                               False, True, -1, -1, 0.0, False, 0, None)
    assert tuple(out.shape) == (6, 8, 128) and out.dtype == torch.float16
    assert tuple(lse.shape) == (8, 6) and lse.dtype == torch.float32


def test_fa2_fork_interface_rejects_unsupported():
    """The argument checks of kernels_vllm_fa2_fork's Python entry points
    (reference interface.py:200-217, 367-372) and this build's explicit
    limits; all raise before any kernel is reached."""
    from sub0_amd.cda import kernels_vllm_fa2_fork as F
    q = torch.zeros(4, 8, 128, dtype=torch.float16)
    k = torch.zeros(4, 2, 128, dtype=torch.float16)
    cu = torch.tensor([0, 4], dtype=torch.int32)
    with pytest.raises(ValueError, match="must be provided"):
        F.flash_attn_varlen_func(q, k, k, 4, cu, 4)
    with pytest.raises(ValueError, match="cannot both"):
        F.flash_attn_varlen_func(q, k, k, 4, cu, 4, cu_seqlens_k=cu, seqused_k=cu[1:])
    with pytest.raises(ValueError, match="block_table"):
        F.flash_attn_varlen_func(q, k, k, 4, cu, 4, cu_seqlens_k=cu, block_table=cu)
    with pytest.raises(ValueError, match="fa_version"):
        F.flash_attn_varlen_func(q, k, k, 4, cu, 4, cu_seqlens_k=cu, fa_version=3)
    with pytest.raises(NotImplementedError, match="dropout"):
        F.flash_attn_varlen_func(q, k, k, 4, cu, 4, cu_seqlens_k=cu, dropout_p=0.1)
    with pytest.raises(ValueError, match="exactly two"):
        F.flash_attn_varlen_func(q, k, k, 4, cu, 4, cu_seqlens_k=cu, window_size=(1,))
    ki = torch.zeros(4, 2, 64, dtype=torch.uint8)
    kn = torch.zeros(4, 2)
    cb = torch.zeros(16)
    with pytest.raises(ValueError, match="must be provided"):
        F.flash_attn_varlen_compressed_kv_fused_func(q, ki, kn, ki, kn, cb, cb, 4, cu, 4)
    with pytest.raises(ValueError, match="seqused_k"):
        F.flash_attn_varlen_compressed_kv_fused_func(q, ki, kn, ki, kn, cb, cb, 4, cu, 4,
                                                     block_table=cu)
    with pytest.raises(ValueError, match="3D or 4D"):
        F.dequantize_compressed_kv(ki[0], kn[0], ki[0], kn[0], cb, cb)
    with pytest.raises(ImportError):
        F.register_vllm_backend()


def test_native_torch_library_loads_standalone():
    """libcda_hip_torch.so is a TORCH_LIBRARY build: a process that never
    imports this package gets both namespaces from torch.ops.load_library
    alone (as the reference's load_torch_ops_library does,
    _prebuilt_loader.py:69-80), with the in-place schemas, the C++ argument
    checks (TypeError / ValueError before any GPU work) and Meta kernels."""
    import subprocess
    import sys
    from pathlib import Path
    lib = Path(__file__).resolve().parents[1] / "sub0_amd" / "_lib" / "libcda_hip_torch.so"
    code = f"""
import torch
torch.ops.load_library({str(lib)!r})
s = str(torch.ops.cda_hip.decode.default._schema)
assert s.startswith("cda_hip::decode(") and "Tensor(a!) out" in s, s
assert "Tensor(a!)? out" in str(torch.ops._cda_vllm_fa2_fork_C.varlen_fwd.default._schema)
q = torch.zeros(2, 32, 128, dtype=torch.float32)
try:
    torch.ops.cda_hip.hadamard128(q, q, 1.0)
except (TypeError, ValueError, NotImplementedError, RuntimeError) as e:
    print("ERR", type(e).__name__)
with torch.device("meta"):
    kv = torch.empty(64, 8, 144, dtype=torch.uint8)
    bt = torch.empty(2, 4, dtype=torch.int32)
    sl = torch.empty(2, dtype=torch.int32)
    cb = torch.empty(16)
    k, v = torch.ops.cda_hip.paged_to_dense(kv, bt, sl, cb, cb, 16, 40)
    assert k.shape == (80, 8, 128) and k.dtype == torch.float16
print("OK")
"""
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-2000:]
    # A CPU tensor has no CUDA kernel: the dispatcher refuses it (no CPU path).
    assert "ERR NotImplementedError" in r.stdout and r.stdout.strip().endswith("OK"), r.stdout
