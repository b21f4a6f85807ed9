"""GPU: the custom ops (torch.ops.gfx906_fa.*) run the same kernels as the
op-module functions, bit for bit; torch.library.opcheck validates their
schemas and fake implementations against real calls; an aot_eager
torch.compile of a decode step (functionalised in-place ops) matches eager.

The op forms follow the reference's extension module
(extension/gfx906_fa.cpp:660-690); the attention results themselves are
checked against the oracle in tests/test_gpu_attention.py.
"""
import math

import numpy as np
import pytest
import torch

import gfx906_fa
import gfx906_fa_workloads as W
from gpu_common import announce, need_gpu

pytestmark = pytest.mark.gpu
OPS = torch.ops.gfx906_fa


@pytest.fixture(scope="module")
def batch():
    need_gpu()
    # 3 sequences: a 40-token prefill on a 60-token prefix, a decode, a 5-token verify
    return W.build_batch([100, 300, 77], [40, 1, 5], 8, 2, dtype="f16", seed=11, device="cuda")


def _attn_args(b):
    kp, vp = b.planes()
    return (b.query, kp, vp, b.block_table, b.seq_lens_t, b.qsl_t, b.max_query_len, b.max_seq_len, b.scale)


def test_paged_attention_op_equals_function(batch):
    announce("torch op paged_attention")
    b = batch
    ws = gfx906_fa.new_workspace(gfx906_fa.workspace_size(b.num_seqs, b.num_tokens, b.Hq, b.Hkv,
                                                          b.max_query_len, b.max_seq_len), b.device)
    ref = gfx906_fa.paged_attention(*_attn_args(b), workspace=ws, out_dtype=torch.float32)
    got = OPS.paged_attention(*_attn_args(b), ws, out_dtype=torch.float32)
    got2 = OPS.paged_attention(*_attn_args(b), None)
    out = torch.empty_like(b.query)
    OPS.paged_attention_out(*_attn_args(b), out, ws)
    torch.cuda.synchronize()
    assert torch.equal(got, ref)
    assert torch.equal(got2, ref.to(torch.float16))
    assert torch.equal(out, got2)


def test_cache_write_ops_equal_functions(batch):
    announce("torch op reshape_and_cache_q8_kv / rope_and_cache_q8_kv / quantize / gathers")
    b = batch
    T = 70
    rng = np.random.default_rng(5)
    key = torch.from_numpy(rng.standard_normal((T, 2, 128), dtype=np.float32)).half().cuda()
    val = torch.from_numpy(rng.standard_normal((T, 2, 128), dtype=np.float32)).half().cuda()
    qry = torch.from_numpy(rng.standard_normal((T, 8, 128), dtype=np.float32)).half().cuda()
    slots = torch.from_numpy(rng.permutation(12 * 16)[:T].astype(np.int64)).cuda()
    slots[3] = -1
    c1 = gfx906_fa.new_kv_cache(12, 16, 2, device="cuda")
    c2 = c1.clone()
    gfx906_fa.reshape_and_cache_q8_kv(key, val, slots, c1[:, 0], c1[:, 1])
    OPS.reshape_and_cache_q8_kv(key, val, slots, c2[:, 0], c2[:, 1])
    torch.cuda.synchronize()
    assert torch.equal(c1, c2)
    # fused rotary + write: query and key rotated in place, the caches written
    pos = torch.arange(T, dtype=torch.int64, device="cuda") * 3
    cs = W.rope_cos_sin_cache(256, 128, torch.float16, "cuda")
    q1, k1, q2, k2 = qry.clone(), key.clone(), qry.clone(), key.clone()
    gfx906_fa.rope_and_cache_q8_kv(pos, q1, k1, val, cs, True, slots, c1[:, 0], c1[:, 1])
    OPS.rope_and_cache_q8_kv(pos, q2, k2, val, cs, True, slots, c2[:, 0], c2[:, 1])
    torch.cuda.synchronize()
    assert torch.equal(q1, q2) and torch.equal(k1, k2) and torch.equal(c1, c2)
    assert not torch.equal(q1, qry)
    # dense quantize and the AoS reference write
    assert torch.equal(OPS.quantize_q8_0(key), gfx906_fa.quantize_q8_0(key))
    a1 = torch.zeros(12, 16, 2, 136, dtype=torch.uint8, device="cuda")
    a2 = a1.clone()
    gfx906_fa.reshape_and_cache_q8(key, slots, a1)
    OPS.reshape_and_cache_q8(key, slots, a2)
    torch.cuda.synchronize()
    assert torch.equal(a1, a2)
    # gathers: functional and _out forms
    bt = torch.from_numpy(rng.permutation(12)[:8].astype(np.int32).reshape(2, 4)).cuda()
    sl = torch.tensor([50, 64], dtype=torch.int32, device="cuda")
    vc = torch.from_numpy(rng.standard_normal((12, 16, 2, 128), dtype=np.float32)).half().cuda()
    kr, vr = gfx906_fa.gather_paged_kv_q8(a1, vc, bt, sl, 64)
    ko, vo = OPS.gather_paged_kv_q8(a1, vc, bt, sl, 64)
    kb, vb = torch.empty_like(kr), torch.empty_like(vr)
    OPS.gather_paged_kv_q8_out(a1, vc, bt, sl, 64, kb, vb)
    k3, v3 = gfx906_fa.gather_paged_kv_q8q8(c1[:, 0], c1[:, 1], bt, sl, 64)
    k4, v4 = OPS.gather_paged_kv_q8q8(c1[:, 0], c1[:, 1], bt, sl, 64)
    torch.cuda.synchronize()
    # V rows past seq_len are zeroed; K rows there are left as the (freshly
    # allocated, uninitialised) output held them, so K compares on valid tokens
    assert torch.equal(vo, vr) and torch.equal(vb, vr) and torch.equal(v3, v4)
    for i, n in enumerate(sl.tolist()):
        for kx in (ko, kb):
            assert torch.equal(kx[i, :, :n], kr[i, :, :n])
        assert torch.equal(k4[i, :, :n], k3[i, :, :n])


def test_forward_ops_equal_functions():
    announce("torch op forward / forward_paged_direct")
    need_gpu()
    rng = np.random.default_rng(9)
    B, Hq, Hkv, Sq, Skv = 2, 8, 2, 5, 70
    q = torch.from_numpy(rng.standard_normal((B, Hq, Sq, 128), dtype=np.float32)).cuda()
    kv = torch.from_numpy(rng.standard_normal((B, Hkv, Skv, 128), dtype=np.float32)).half().cuda()
    kq = gfx906_fa.quantize_q8_0(kv)
    v = torch.from_numpy(rng.standard_normal((B, Hkv, Skv, 128), dtype=np.float32)).half().cuda()
    scale = 1 / math.sqrt(128)
    qa = torch.tensor([Skv - Sq, Skv - Sq - 3], dtype=torch.int32, device="cuda")
    assert torch.equal(OPS.forward(q, kq, v, scale, None, None, qa), gfx906_fa.forward(q, kq, v, scale, None, None, qa))
    b = W.build_batch([90, 33], [4, 4], Hq, Hkv, dtype="f16", seed=2, device="cuda")
    kp, vp = b.planes()
    q4 = b.query.view(2, 4, Hq, 128).transpose(1, 2).contiguous()
    r1 = gfx906_fa.forward_paged_direct(q4, kp, vp, b.block_table, b.seq_lens_t, b.scale)
    r2 = OPS.forward_paged_direct(q4, kp, vp, b.block_table, b.seq_lens_t, b.scale)
    torch.cuda.synchronize()
    assert torch.equal(r1, r2)


def test_opcheck(batch):
    """torch.library.opcheck: schema (declared writes), fake implementation
    against the real call, and the autograd / dispatch registrations."""
    announce("torch.library.opcheck")
    b = batch
    kp, vp = b.planes()
    ws = gfx906_fa.new_workspace(gfx906_fa.workspace_size(b.num_seqs, b.num_tokens, b.Hq, b.Hkv,
                                                          b.max_query_len, b.max_seq_len), b.device)
    torch.library.opcheck(OPS.paged_attention.default, _attn_args(b) + (ws,), {"out_dtype": torch.float32})
    out = torch.empty_like(b.query)
    torch.library.opcheck(OPS.paged_attention_out.default, _attn_args(b) + (out, ws))
    key = torch.randn(20, 2, 128, dtype=torch.float16, device="cuda")
    torch.library.opcheck(OPS.quantize_q8_0.default, (key,))
    cache = gfx906_fa.new_kv_cache(4, 16, 2, device="cuda")
    slots = torch.arange(20, dtype=torch.int64, device="cuda")
    torch.library.opcheck(OPS.reshape_and_cache_q8_kv.default, (key, key.clone(), slots, cache[:, 0], cache[:, 1]))


def test_compiled_step_matches_eager(batch):
    """A decode step (cache write of the new tokens + attention) compiled
    with aot_eager - the in-place ops go through functionalisation - gives
    the eager bytes and outputs."""
    announce("torch.compile aot_eager step")
    b = W.build_batch([64, 130, 31], [1, 1, 1], 8, 2, dtype="f16", seed=4, device="cuda")
    kp, vp = b.planes()
    last = torch.from_numpy(np.cumsum(b.seq_lens.astype(np.int64)) - 1).cuda()
    kn = b.key.index_select(0, last).contiguous()
    vn = b.value.index_select(0, last).contiguous()
    sn = b.slot_mapping.index_select(0, last).contiguous()
    ws = gfx906_fa.new_workspace(gfx906_fa.workspace_size(b.num_seqs, b.num_tokens, b.Hq, b.Hkv,
                                                          b.max_query_len, b.max_seq_len), b.device)

    def step(query, cache, kn, vn, sn, bt, sl, qsl, ws):
        torch.ops.gfx906_fa.reshape_and_cache_q8_kv(kn, vn, sn, cache[:, 0], cache[:, 1])
        return torch.ops.gfx906_fa.paged_attention(query, cache[:, 0], cache[:, 1], bt, sl, qsl, 1,
                                                   int(b.max_seq_len), b.scale, ws, out_dtype=torch.float32)

    c_eager = b.kv_cache.clone()
    c_comp = b.kv_cache.clone()
    eager = step(b.query, c_eager, kn, vn, sn, b.block_table, b.seq_lens_t, b.qsl_t, ws)
    torch._dynamo.reset()
    comp = torch.compile(step, fullgraph=True, backend="aot_eager")(
        b.query, c_comp, kn, vn, sn, b.block_table, b.seq_lens_t, b.qsl_t, ws)
    torch.cuda.synchronize()
    torch._dynamo.reset()
    assert torch.equal(c_eager, c_comp)
    assert torch.equal(eager, comp)


def test_paged_attention_out_op_takes_workspace_without_image_room():
    """A 2048-token prompt at 48/8 has room for 64-key tile images in its
    workspace_size(); the out-variant op accepts a workspace of only the
    regions every call needs (plan_info ``img_offset``), as the function
    does, and gives the same output bit for bit (its prefill workgroups then
    dequantize their own tiles); one byte less is refused."""
    announce("torch op paged_attention_out, img_offset workspace")
    b = W.build_batch([2048], [2048], 48, 8, dtype="bf16", seed=13, device="cuda")
    info = gfx906_fa.plan_info(b.num_seqs, b.num_tokens, b.Hq, b.Hkv, b.max_query_len, b.max_seq_len)
    assert info["img_bytes"] > 0
    full = gfx906_fa.new_workspace(info["bytes"], b.device)
    small = gfx906_fa.new_workspace(info["img_offset"], b.device)
    o_full = torch.empty_like(b.query)
    o_small = torch.empty_like(b.query)
    OPS.paged_attention_out(*_attn_args(b), o_full, full)
    OPS.paged_attention_out(*_attn_args(b), o_small, small)
    torch.cuda.synchronize()
    assert torch.equal(o_full, o_small)
    short = gfx906_fa.new_workspace(info["img_offset"] - 256, b.device)
    with pytest.raises(RuntimeError, match="workspace needs"):
        OPS.paged_attention_out(*_attn_args(b), o_small, short)
