"""CPU: the vLLM plugin surface against the offline vllm stub.

Follows tests/test_backend.py:30-57 of the reference (registration as
CUSTOM, kv-cache shape equal to Triton's) and the error behaviour of
extension/gfx906_fa_backend.py:247-257, 463-468.  vLLM itself is absent, so
vLLM-side behaviour is unpinned; these tests pin this backend's side."""
import os

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


def _vllm_style_cache(backend, NB, bs, Hkv, D, cache_dtype, model_dtype):
    """What vLLM's allocator does with a backend: one raw int8 buffer of
    page_size x num_blocks bytes, viewed in the cache dtype and the backend's
    shape."""
    page = backend.get_kv_cache_page_size_bytes(bs, Hkv, D, cache_dtype, model_dtype)
    raw = torch.zeros(page * NB, dtype=torch.int8)
    dt = torch.uint8 if cache_dtype == "q8_0" else model_dtype
    return raw.view(dt).view(backend.get_kv_cache_shape(NB, bs, Hkv, D, cache_dtype)), page


@pytest.mark.parametrize("bs", [16, 32, 64])
def test_q8_0_pages_hold_exactly_the_planes(bs):
    """The "q8_0" cache dtype: pages of 272 B per token and kv-head, whose
    planes sit at the same offsets inside the page as in an fp16 page (so the
    kernels see the same bytes; only the page stride shrinks)."""
    from gfx906_fa_backend import Gfx906FABackend, Gfx906FAImpl
    from gfx906_fa_paged import q8_planes
    NB, Hkv, D = 6, 8, 128
    assert "q8_0" in Gfx906FABackend.supported_kv_cache_dtypes
    q8, page_q8 = _vllm_style_cache(Gfx906FABackend, NB, bs, Hkv, D, "q8_0", torch.float16)
    f16, page_f16 = _vllm_style_cache(Gfx906FABackend, NB, bs, Hkv, D, "auto", torch.float16)
    assert page_q8 == bs * Hkv * 2 * (D // 32 * 34)          # 272 B per token and kv-head
    assert page_f16 == bs * Hkv * 2 * D * 2 and page_f16 * 136 == page_q8 * 256
    assert q8.shape == (NB, 2, Hkv, bs // 16, 2176)
    kq, vq = q8_planes(q8, Hkv, D, block_size=bs)
    kf, vf = q8_planes(f16, Hkv, D, block_size=bs)
    assert kq.shape == kf.shape == vq.shape == vf.shape == (NB, Hkv, bs // 16 * 2176)
    assert kq.stride() == (page_q8, bs // 16 * 2176, 1) and vq.stride() == kq.stride()
    for (k, v, base, page) in ((kq, vq, q8.data_ptr(), page_q8), (kf, vf, f16.data_ptr(), page_f16)):
        assert k.data_ptr() - base == 0
        assert v.data_ptr() - base == Hkv * bs // 16 * 2176     # V plane after every K plane
    # every byte of a q8_0 page belongs to exactly one plane
    marks = torch.zeros(page_q8 * NB, dtype=torch.uint8)
    mv = marks.view(q8.shape)
    km, vm = q8_planes(mv, Hkv, D)
    km.add_(1)
    vm.add_(2)
    assert set(marks.unique().tolist()) == {1, 2}
    assert int((marks == 1).sum()) == int((marks == 2).sum()) == NB * bs * Hkv * 136
    Gfx906FAImpl(8, 128, 0.1, 1, None, None, "q8_0")          # accepted
    with pytest.raises(NotImplementedError):
        Gfx906FAImpl(8, 128, 0.1, 1, None, None, "fp8")
    with pytest.raises(ValueError):
        Gfx906FABackend.get_kv_cache_shape(NB, bs, Hkv, 64, "q8_0")
    with pytest.raises(RuntimeError):
        q8_planes(q8, Hkv, D, block_size=2 * bs)


def test_graph_support_and_workspace_bound():
    """The builder declares graph support for uniform batches; the workspace
    bound covers every batch of up to max_num_seqs sequences and
    max_num_tokens tokens: uniform and non-uniform query lengths (both decode
    classes plus prefill rows in one batch), chunked-prefill token budgets,
    and kv-head counts that do not divide the CU count."""
    import random
    import gfx906_fa
    from gfx906_fa_backend import Gfx906FAMetadataBuilder, workspace_upper_bound
    from vllm.v1.attention.backend import AttentionCGSupport
    assert Gfx906FAMetadataBuilder._cudagraph_support == AttentionCGSupport.UNIFORM_BATCH
    rng = random.Random(0)
    heads = ((48, 8), (6, 1), (32, 32), (12, 3), (10, 5), (36, 6), (40, 10), (48, 12), (64, 1), (128, 1),
             (8, 1), (96, 3))
    for hq, hkv in heads:
        for max_seqs, max_tokens in ((1, 1), (1, 8192), (7, 7), (7, 4096), (256, 256), (256, 8192),
                                     (256, 65536), (1024, 16384)):
            bound = workspace_upper_bound(max_seqs, max_tokens, [(hq, hkv)])
            assert bound == gfx906_fa.workspace_bound(max_seqs, max_tokens, hq, hkv) > 0
            shapes = []
            for n in {1, max(1, max_seqs // 2), max_seqs}:
                for mq in (1, 2, 5, 6, 7, 8, 16, 2048):
                    if n * mq <= max_tokens:
                        shapes.append((n, n * mq, mq))          # uniform
                        if n > 1:
                            shapes.append((n, n * mq - 1, mq))  # one sequence a token short
                if n <= max_tokens:
                    # one long prefill chunk with n - 1 decode / verify sequences
                    for extra in (1, 5, 6):
                        big = max_tokens - extra * (n - 1)
                        if big >= 1:
                            shapes.append((n, big + extra * (n - 1), big))
            for _ in range(40):
                n = rng.randint(1, max_seqs)
                if n > max_tokens:
                    continue
                T = rng.randint(n, max_tokens)
                shapes.append((n, T, rng.randint(1, T - n + 1)))
            info = gfx906_fa.workspace_bound_info(max_seqs, max_tokens, hq, hkv)
            assert info["regions"] + info["img_bytes"] == bound
            for n, T, mq in shapes:
                # long and short contexts: the decode classes differ (48-row
                # tiles only with enough sub-pages per workgroup)
                for msl in (1 << 17, 2048):
                    need = gfx906_fa.workspace_size(n, T, hq, hkv, mq, msl)
                    assert need <= bound, (hq, hkv, max_seqs, max_tokens, n, T, mq, msl, need, bound)
                    # the regions alone run every call (the image room is optional)
                    reg = gfx906_fa.plan_info(n, T, hq, hkv, mq, msl)["img_offset"]
                    assert reg <= info["regions"], (hq, hkv, max_seqs, max_tokens, n, T, mq, msl)
    # several layer shapes: the largest bound
    both = workspace_upper_bound(64, 4096, [(48, 8), (6, 1)])
    assert both == max(gfx906_fa.workspace_bound(64, 4096, 48, 8), gfx906_fa.workspace_bound(64, 4096, 6, 1))


def test_bound_image_room_follows_max_model_len_and_the_cap(monkeypatch):
    """The image part of the bound shrinks with max_model_len and is capped
    by GFX906_FA_IMAGE_ROOM_MB; the regions part is independent of both."""
    import gfx906_fa
    from gfx906_fa_backend import image_room_bytes, workspace_upper_bound
    full = gfx906_fa.workspace_bound_info(16, 8192, 48, 8)
    short = gfx906_fa.workspace_bound_info(16, 8192, 48, 8, max_seq_len=4096)
    # up to 16 prefill sequences of 4096 keys: 64 tiles x 8 kv-heads x 35840 B each
    assert full["img_bytes"] == 1 << 30 and short["img_bytes"] == 16 * 64 * 8 * 35840
    assert short["regions"] == full["regions"]
    monkeypatch.delenv("GFX906_FA_IMAGE_ROOM_MB", raising=False)
    assert image_room_bytes() == 256 << 20
    monkeypatch.setenv("GFX906_FA_IMAGE_ROOM_MB", "0")
    assert image_room_bytes() == 0
    assert workspace_upper_bound(16, 8192, [(48, 8)], -1, 0) == full["regions"]
    assert workspace_upper_bound(16, 8192, [(48, 8)], -1, 100 << 20) == full["regions"] + (100 << 20)
    assert workspace_upper_bound(16, 8192, [(48, 8)], 4096, 1 << 30) == short["regions"] + short["img_bytes"]


def test_profiling_forward_reserves_the_bound(monkeypatch):
    """vLLM sizes the KV cache from the memory its profiling run used, so the
    profiling forward (attn_metadata None) reserves the workspace bound of
    the scheduler limits (taken from the current vLLM config at model
    construction) on the device."""
    import types
    import gfx906_fa_backend as GB
    from gfx906_fa_backend import Gfx906FAImpl
    from vllm.config import set_current_vllm_config
    monkeypatch.setattr(Gfx906FAImpl, "_limits", None)
    monkeypatch.setattr(Gfx906FAImpl, "_layer_heads", set())
    asked = []
    monkeypatch.setattr(Gfx906FAImpl, "reserve_workspace",
                        classmethod(lambda cls, n, dev: asked.append((n, dev.type))))
    cfg = types.SimpleNamespace(scheduler_config=types.SimpleNamespace(max_num_seqs=64, max_num_batched_tokens=4096),
                                model_config=types.SimpleNamespace(max_model_len=32768))
    with set_current_vllm_config(cfg):
        impl = Gfx906FAImpl(48, 128, 0.1, 8, None, None, "auto")
    assert Gfx906FAImpl._limits == (64, 4096, 32768)
    out = torch.ones(3, 48 * 128)
    fake_q = types.SimpleNamespace(device=torch.device("cuda"))
    assert impl.forward(None, fake_q, None, None, None, None, output=out) is out and not out.any()
    assert asked == [(Gfx906FAImpl.bound_bytes({(48, 8)}, (64, 4096, 32768)), "cuda")]
    assert asked[0][0] == GB.workspace_upper_bound(64, 4096, [(48, 8)], 32768, GB.image_room_bytes())


def test_builder_reserves_the_bound_and_retires_workspaces(monkeypatch):
    """The builder reserves the bound for the scheduler limits and the layer
    shapes; a larger request later replaces the workspace.  Before any graph
    capture the old one is freed; after a capture it is kept alive (a
    captured graph may still write into it)."""
    import types
    import gfx906_fa
    import gfx906_fa_backend as GB
    from gfx906_fa_backend import Gfx906FAImpl, Gfx906FAMetadataBuilder, workspace_upper_bound
    from vllm.v1.kv_cache_interface import AttentionSpec
    made = []

    def fake_new_workspace(nbytes, device):
        t = torch.empty(max(int(nbytes), 256), dtype=torch.uint8)
        made.append(t)
        return t

    monkeypatch.setattr(gfx906_fa, "new_workspace", fake_new_workspace)
    monkeypatch.setattr(Gfx906FAImpl, "_workspace", None)
    monkeypatch.setattr(Gfx906FAImpl, "_retired", [])
    monkeypatch.setattr(Gfx906FAImpl, "_captured", False)
    monkeypatch.setattr(Gfx906FAImpl, "_layer_heads", set())
    monkeypatch.setattr(Gfx906FAImpl, "_limits", None)
    Gfx906FAImpl(48, 128, 0.1, 8, None, None, "auto")
    Gfx906FAImpl(6, 128, 0.1, 1, None, None, "auto")
    cfg = types.SimpleNamespace(scheduler_config=types.SimpleNamespace(max_num_seqs=128,
                                                                       max_num_batched_tokens=8192))
    # a CPU device never reserves (no GPU here): the bound is reserved for cuda only
    Gfx906FAMetadataBuilder(AttentionSpec(block_size=16, num_kv_heads=8), ["l0"], cfg, torch.device("cpu"))
    assert Gfx906FAImpl._workspace is None
    want = workspace_upper_bound(128, 8192, [(48, 8), (6, 1)])
    cpu = torch.device("cpu")
    first = Gfx906FAImpl.reserve_workspace(want, cpu)
    assert first.numel() >= want and Gfx906FAImpl._retired == []
    assert Gfx906FAImpl.reserve_workspace(want // 2, cpu) is first      # never shrinks
    second = Gfx906FAImpl.reserve_workspace(want + 1, cpu)
    assert second is not first and second.numel() >= want + want // 4  # grows by a quarter at least
    assert Gfx906FAImpl._retired == []                                   # no capture yet: freed
    assert GB.Gfx906FAImpl._workspace is second
    # a capture from the builder: replaced workspaces now stay alive
    from vllm.v1.attention.backend import CommonAttentionMetadata
    b = Gfx906FAMetadataBuilder(AttentionSpec(block_size=16, num_kv_heads=8), ["l0"], cfg, cpu)
    md = CommonAttentionMetadata(query_start_loc=torch.tensor([0, 1], dtype=torch.int32),
                                 seq_lens=torch.tensor([5], dtype=torch.int32), num_reqs=1,
                                 num_actual_tokens=1, max_query_len=1, max_seq_len=5,
                                 block_table_tensor=torch.zeros(1, 1, dtype=torch.int32),
                                 slot_mapping=torch.zeros(1, dtype=torch.int64))
    b.build_for_cudagraph_capture(md)
    assert Gfx906FAImpl._captured
    third = Gfx906FAImpl.reserve_workspace(second.numel() + 1, cpu)
    assert third is not second and Gfx906FAImpl._retired == [second]


def test_forward_debug_log_records_the_call_and_its_failure(tmp_path, monkeypatch):
    """GFX906_FA_FWD_DEBUG: the call's shapes are logged before the launch and
    the error after it, and the error still propagates.  CPU tensors make the
    op fail its device check, so no GPU is needed."""
    import os
    import gfx906_fa_paged as P
    monkeypatch.setattr(P, "_DBG", True)
    monkeypatch.setattr(P, "_DBG_DIR", str(tmp_path / "dbg"))
    q = torch.zeros(2, 8, 128, dtype=torch.float16)
    kp = torch.zeros(4, 2, 2176, dtype=torch.uint8)
    bt = torch.zeros(2, 1, dtype=torch.int32)
    sl = torch.ones(2, dtype=torch.int32)
    cu = torch.tensor([0, 1, 2], dtype=torch.int32)
    with pytest.raises(RuntimeError):
        P.forward_paged(q, kp, kp, bt, sl, cu, 1, 1)
    lines = (tmp_path / "dbg" / f"fwd-{os.getpid()}.log").read_text().splitlines()
    assert len(lines) == 2
    assert "forward_paged VARLEN: num_tokens=2 Hq=8 Hkv=2 D=128 num_seqs=2" in lines[0]
    assert "forward_paged FAILED" in lines[1]


def test_forward_debug_log_off_by_default(tmp_path, monkeypatch):
    import gfx906_fa_paged as P
    assert P._DBG == (os.environ.get("GFX906_FA_FWD_DEBUG", "0") == "1")
    monkeypatch.setattr(P, "_DBG", False)
    monkeypatch.setattr(P, "_DBG_DIR", str(tmp_path / "dbg"))
    P._fwdlog("x")
    assert not (tmp_path / "dbg").exists()
