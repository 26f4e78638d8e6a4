"""Host-side checks of the vLLM backend glue (no GPU, no vLLM): slot layout,
cache reinterpretation, the decode/prefill split, backend descriptor, impl
argument checks and dispatch (cda_attn_v2.py:44-78, 366-383, 552-748)."""
import importlib

import pytest
import torch

from sub0_amd.cda.kernels_cuda.vllm_integration import cda_attn_v2 as A


def test_layout_constants():
    assert (A._DATA_BYTES_PER_TOKEN, A._BYTES_PER_TOKEN) == (136, 144)
    assert A._SLOT_FP16_ELEMS_COMPACT == 72


@pytest.mark.parametrize("last,width", [(72, 144), (256, 512)])
def test_as_uint8_cache_views_same_storage(last, width):
    c = torch.zeros(3, 16, 8, last, dtype=torch.float16)
    u = A._as_uint8_cache(c)
    assert u.shape == (3, 16, 8, width) and u.dtype == torch.uint8
    assert u.data_ptr() == c.data_ptr()
    u[1, 2, 3, 5] = 7                            # a write lands in the fp16 buffer
    assert c.view(torch.uint8).view(3, 16, 8, width)[1, 2, 3, 5] == 7
    assert A._as_uint8_cache(u) is u


def test_as_uint8_cache_rejects_other_widths():
    with pytest.raises(ValueError):
        A._as_uint8_cache(torch.zeros(1, 16, 8, 64, dtype=torch.float16))


@pytest.mark.parametrize("qs,max_q,expect", [
    ([0, 1, 2, 3], 1, (3, 0, 3, 0)),            # pure decode
    ([0, 5, 9], 5, (0, 2, 0, 9)),               # pure prefill
    ([0, 1, 2, 7, 20], 13, (2, 2, 2, 18)),      # decode first, then prefill
    ([0, 1, 1, 4], 3, (2, 1, 1, 3)),            # an empty request counts as decode
])
def test_split_counts(qs, max_q, expect):
    n = len(qs) - 1
    got = A._split_counts_from_query_start(torch.tensor(qs, dtype=torch.int32), n, qs[-1], max_q)
    assert got == expect
    assert A._split_counts_from_query_start(qs, n, qs[-1], max_q) == expect


def test_backend_descriptor_without_vllm():
    Backend, Impl, Builder, Meta = A.get_backend_classes()
    assert A.get_backend_classes()[0] is Backend
    assert Backend.get_name() == "CDA"
    assert Backend.get_impl_cls() is Impl and Backend.get_builder_cls() is Builder
    assert Backend.get_kv_cache_shape(10, 16, 8, 128) == (10, 16, 8, 72)
    with pytest.raises(ValueError):
        Backend.get_kv_cache_shape(10, 16, 8, 64)
    assert Backend.get_supported_head_sizes() == [128]
    assert [int(x) for x in Backend.get_supported_kernel_block_sizes()] == [16]
    assert Backend.supported_dtypes == [torch.float16] and Backend.accept_output_buffer


def test_swap_and_copy_blocks():
    Backend = A.get_backend_classes()[0]
    src = torch.arange(4 * 6, dtype=torch.float16).view(4, 6)
    dst = torch.zeros_like(src)
    Backend.swap_blocks(src, dst, torch.tensor([[0, 3], [2, 1]]))
    assert torch.equal(dst[3], src[0]) and torch.equal(dst[1], src[2])
    assert not dst[0].any() and not dst[2].any()
    c = src.clone()
    Backend.copy_blocks([c], torch.tensor([[1, 0]]))
    assert torch.equal(c[0], src[1])


def test_impl_argument_checks():
    Impl = A.get_backend_classes()[1]
    impl = Impl(32, 128, 0.088, num_kv_heads=8)
    assert impl.group_size == 4 and impl.scale == pytest.approx(0.088)
    assert Impl(64, 128, 0.1, num_kv_heads=8).group_size == 8
    for kw in ({"num_kv_heads": 16}, {"num_kv_heads": 8, "alibi_slopes": [1.0]},
               {"num_kv_heads": 8, "sliding_window": 512},
               {"num_kv_heads": 8, "attn_type": "encoder"}):
        with pytest.raises(NotImplementedError):
            Impl(32, 128, 0.1, **kw)


def _meta(**kw):
    base = dict(num_actual_tokens=2, num_reqs=2, max_query_len=1, max_seq_len=4,
                query_start_loc=torch.tensor([0, 1, 2], dtype=torch.int32),
                seq_lens=torch.tensor([4, 4], dtype=torch.int32),
                block_table=torch.zeros(2, 1, dtype=torch.int32),
                slot_mapping=torch.tensor([3, 19]))
    base.update(kw)
    return A.CDAv2AttentionMetadata(**base)


def test_forward_guards_and_routing(monkeypatch):
    Impl = A.get_backend_classes()[1]
    impl = Impl(32, 128, 0.1, num_kv_heads=8)
    q = torch.zeros(2, 32, 128, dtype=torch.float16)
    cache = torch.zeros(2, 16, 8, 72, dtype=torch.float16)
    out = torch.ones(2, 32 * 128, dtype=torch.float16)
    with pytest.raises(ValueError):
        impl.forward(None, q, q, q, cache, _meta(), None)
    with pytest.raises(NotImplementedError):
        impl.forward(None, q, q, q, cache, _meta(), out, output_scale=torch.ones(1))
    assert not impl.forward(None, q, q, q, cache, None, out).any()
    with pytest.raises(NotImplementedError):
        impl.forward(None, q, q, q, cache, _meta(dcp_world_size=2), out)

    seen = []
    monkeypatch.setattr(impl, "_forward_decode", lambda *a: seen.append("decode"))
    monkeypatch.setattr(impl, "_forward_prefill", lambda *a: seen.append("prefill"))
    monkeypatch.setattr(impl, "_forward_mixed_prefill_decode", lambda *a: seen.append("mixed"))
    impl.forward(None, q, q, q, cache, _meta(), out)
    md = _meta(max_query_len=2, num_actual_tokens=4,
               query_start_loc=torch.tensor([0, 2, 4], dtype=torch.int32))
    impl.forward(None, q, q, q, cache, md, out)
    assert (md.num_decodes, md.num_prefills, md.num_prefill_tokens) == (0, 2, 4)
    md = _meta(max_query_len=3, num_actual_tokens=4,
               query_start_loc=torch.tensor([0, 1, 4], dtype=torch.int32))
    impl.forward(None, q, q, q, cache, md, out)
    assert seen == ["decode", "prefill", "mixed"]


def test_prefill_route_errors(monkeypatch):
    Impl = A.get_backend_classes()[1]
    impl = Impl(32, 128, 0.1, num_kv_heads=8)
    q = torch.zeros(4, 32, 128, dtype=torch.float16)
    cache = A._as_uint8_cache(torch.zeros(2, 16, 8, 72, dtype=torch.float16))
    md = _meta(max_query_len=2, num_actual_tokens=4)
    monkeypatch.setenv("CDA_PREFILL_BACKEND", "hmma")
    with pytest.raises(NotImplementedError):
        impl._forward_prefill(q, q, q, q, md, cache)
    monkeypatch.setenv("CDA_PREFILL_BACKEND", "fa2_rawkv")
    with pytest.raises(ValueError, match="fresh prefill key/value"):
        impl._forward_prefill(q, None, None, q, md, cache)
    monkeypatch.setenv("CDA_PREFILL_BACKEND", "fa2_cda_fused")
    with pytest.raises(NotImplementedError):
        impl._forward_prefill(q, q, q, q, _meta(max_query_len=0), cache)


def test_builder_builds_metadata_from_common():
    Builder = A.get_backend_classes()[2]
    bld = Builder(None, ["l0"], None, torch.device("cpu"))

    class Common:
        num_actual_tokens = 6
        num_reqs = 3
        max_query_len = 4
        max_seq_len = 40
        query_start_loc = torch.tensor([0, 1, 2, 6], dtype=torch.int32)
        seq_lens = torch.tensor([10, 40, 4], dtype=torch.int32)
        block_table_tensor = torch.zeros(3, 3, dtype=torch.int32)
        slot_mapping = torch.arange(6)
        causal = True

    md = bld.build(0, Common())
    assert (md.num_decodes, md.num_prefills, md.num_decode_tokens, md.num_prefill_tokens) \
        == (2, 1, 2, 4)
    assert md.block_table is Common.block_table_tensor and md.dcp_world_size == 1
    assert Builder.get_cudagraph_support(None, None) == "uniform_batch"


def test_vllm_entry_points_need_vllm():
    if importlib.util.find_spec("vllm") is not None:
        pytest.skip("vLLM is installed")
    with pytest.raises(ModuleNotFoundError):
        A.register_backend("CDA")
    with pytest.raises(ModuleNotFoundError):
        A.enable_cda_memory_saving()
    from sub0_amd.cda.vllm_integration import _backend_eager
    assert _backend_eager.CDAv2AttentionBackend is A.get_backend_classes()[0]
    from sub0_amd.cda import vllm_plugin
    with pytest.raises(ModuleNotFoundError):
        vllm_plugin.register_cda_v2()
