"""CPU: the vLLM plugin surface against the offline vllm stub.

Follows tests/test_backend.py:30-57 of the reference (registration as
CUSTOM, kv-cache shape equal to Triton's) and the error behaviour of
extension/gfx906_fa_backend.py:247-257, 463-468.  vLLM itself is absent, so
vLLM-side behaviour is unpinned; these tests pin this backend's side."""
import pytest
import torch


def test_registration_as_custom():
    import gfx906_fa_backend
    from vllm.v1.attention.backends.registry import AttentionBackendEnum
    assert AttentionBackendEnum.CUSTOM.get_class() is gfx906_fa_backend.Gfx906FABackend


def test_backend_static_surface():
    from gfx906_fa_backend import Gfx906FABackend, Gfx906FAImpl
    from vllm.v1.attention.backend import AttentionType
    assert Gfx906FABackend.get_name() == "CUSTOM"
    assert Gfx906FABackend.accept_output_buffer is True
    assert Gfx906FABackend.forward_includes_kv_cache_update is False
    # identical to TritonAttentionBackend.get_kv_cache_shape
    assert Gfx906FABackend.get_kv_cache_shape(128, 16, 8, 128, "auto") == (128, 2, 16, 8, 128)
    with pytest.raises(ValueError):
        Gfx906FABackend.get_kv_cache_shape(128, 24, 8, 128)
    assert Gfx906FABackend.supports_head_size(128) and not Gfx906FABackend.supports_head_size(64)
    assert Gfx906FABackend.supports_block_size(32) and not Gfx906FABackend.supports_block_size(24)
    assert Gfx906FABackend.supports_attn_type(AttentionType.DECODER)
    assert not Gfx906FABackend.supports_attn_type(AttentionType.ENCODER)
    assert torch.bfloat16 in Gfx906FABackend.supported_dtypes
    assert Gfx906FABackend.get_impl_cls() is Gfx906FAImpl


@pytest.mark.parametrize("kw", [dict(alibi_slopes=[1.0]), dict(sliding_window=128),
                                dict(logits_soft_cap=30.0), dict(sinks=torch.zeros(1))])
def test_unsupported_features_raise(kw):
    from gfx906_fa_backend import Gfx906FAImpl
    args = dict(num_heads=8, head_size=128, scale=0.1, num_kv_heads=1, alibi_slopes=None,
                sliding_window=None, kv_cache_dtype="auto")
    args.update(kw)
    with pytest.raises(NotImplementedError):
        Gfx906FAImpl(**args)


def test_profiling_run_zero_fills():
    from gfx906_fa_backend import Gfx906FAImpl
    impl = Gfx906FAImpl(8, 128, 0.1, 1, None, None, "auto")
    out = torch.ones(3, 8 * 128)
    r = impl.forward(None, torch.zeros(3, 8, 128), None, None, torch.zeros(1), None, output=out)
    assert r is out and not out.any()
    with pytest.raises(NotImplementedError):
        impl.forward(None, None, None, None, None, None, output=out, output_scale=torch.ones(1))


def test_metadata_builder():
    from gfx906_fa_backend import Gfx906FAMetadataBuilder
    from vllm.v1.attention.backend import CommonAttentionMetadata
    from vllm.v1.kv_cache_interface import AttentionSpec
    b = Gfx906FAMetadataBuilder(AttentionSpec(block_size=16), ["l0"], None, torch.device("cpu"))
    cm = CommonAttentionMetadata(query_start_loc=torch.tensor([0, 1, 3], dtype=torch.int32),
                                 seq_lens=torch.tensor([5, 9], dtype=torch.int32), num_reqs=2,
                                 num_actual_tokens=3, max_query_len=2, max_seq_len=9,
                                 block_table_tensor=torch.zeros(2, 1, dtype=torch.int32),
                                 slot_mapping=torch.zeros(3, dtype=torch.int64))
    md = b.build(0, cm)
    assert md.num_actual_tokens == 3 and md.max_seq_len == 9 and not md.use_cascade
    assert b.build(4, cm).use_cascade


def test_q8_planes_inside_vllm_pages():
    from gfx906_fa_paged import q8_planes
    NB, bs, Hkv = 5, 32, 4
    kv = torch.zeros((NB, 2, bs, Hkv, 128), dtype=torch.float16)
    k, v = q8_planes(kv, Hkv, 128)
    page = 2 * bs * Hkv * 128 * 2
    assert k.shape == (NB, Hkv, 2 * 2176) and v.shape == k.shape
    assert k.stride() == (page, 2 * 2176, 1) and v.stride() == k.stride()
    base = kv.data_ptr()
    assert k.data_ptr() == base and v.data_ptr() == base + Hkv * 2 * 2176
    assert (v.data_ptr() - base + v.shape[1] * v.stride(1)) <= page
    with pytest.raises(RuntimeError):
        q8_planes(torch.zeros((NB, 2, bs, Hkv, 64), dtype=torch.float16), Hkv, 64)
    planar = torch.zeros((NB, 2, Hkv, 2176), dtype=torch.uint8)
    k2, v2 = q8_planes(planar, Hkv, 128)
    assert k2.data_ptr() == planar.data_ptr()


def test_graph_support_and_workspace_bound():
    """The builder declares graph support for uniform batches; the workspace
    it reserves up front covers every batch of up to max_num_seqs sequences,
    whatever the heads, query length or context."""
    import gfx906_fa
    from gfx906_fa_backend import Gfx906FAMetadataBuilder, workspace_upper_bound
    from vllm.v1.attention.backend import AttentionCGSupport
    assert Gfx906FAMetadataBuilder._cudagraph_support == AttentionCGSupport.UNIFORM_BATCH
    for max_seqs in (1, 7, 256):
        bound = workspace_upper_bound(max_seqs)
        for n in {1, max_seqs // 2 or 1, max_seqs}:
            for Hq, Hkv in ((48, 8), (6, 1), (32, 32)):
                for mq in (1, 4, 5, 16, 2048):
                    assert gfx906_fa.workspace_size(n, n * mq, Hq, Hkv, mq, 1 << 17) <= bound
