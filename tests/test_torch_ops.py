"""CPU: the op module's PyTorch custom ops (torch.ops.gfx906_fa.*).

The reference exposes its ops through a torch extension module
(extension/gfx906_fa.cpp:660-690).  Here the same functions are registered as
torch.library custom ops over the C ABI, with fake implementations, so that
torch.compile traces them as opaque graph nodes.  These tests run without a
GPU: schemas, fake-tensor shape propagation on fake CUDA tensors, and a
fullgraph torch.compile capture whose backend records the graph and never
runs the kernels.  tests/test_gpu_torch_ops.py runs the ops on the GPU.
"""
import torch
from torch._subclasses.fake_tensor import FakeTensorMode

import gfx906_fa

OPS = torch.ops.gfx906_fa

# in-place (written) arguments each op declares
MUTATES = {
    "quantize_q8_0": set(),
    "reshape_and_cache_q8": {"k_cache_q8"},
    "gather_paged_kv_q8": set(),
    "gather_paged_kv_q8_out": {"k_out", "v_out"},
    "forward": set(),
    "forward_paged_direct": set(),
    "reshape_and_cache_q8_kv": {"key_cache", "value_cache"},
    "rope_and_cache_q8_kv": {"query", "key", "key_cache", "value_cache"},
    "gather_paged_kv_q8q8": set(),
    "paged_attention": {"workspace"},
    "paged_attention_out": {"out", "workspace", "key_cache", "value_cache"},
}


def test_every_op_registered_with_its_writes():
    assert set(gfx906_fa.TORCH_OPS) == set(MUTATES)
    for name, writes in MUTATES.items():
        schema = getattr(OPS, name).default._schema
        got = {a.name for a in schema.arguments if a.alias_info is not None and a.alias_info.is_write}
        assert got == writes, (name, got)
        # functional ops return fresh tensors, in-place ones nothing
        if name in ("quantize_q8_0", "forward", "forward_paged_direct", "paged_attention"):
            assert len(schema.returns) == 1
        elif name in ("gather_paged_kv_q8", "gather_paged_kv_q8q8"):
            assert len(schema.returns) == 2
        else:
            assert len(schema.returns) == 0


def _fake(mode, shape, dtype):
    with mode:
        return torch.empty(shape, dtype=dtype, device="cuda")


def test_fake_shapes():
    mode = FakeTensorMode()
    f = lambda shape, dtype: _fake(mode, shape, dtype)  # noqa: E731
    with mode:
        # quantize: last dim D -> D/32*34 bytes
        k = f((7, 3, 128), torch.float16)
        assert OPS.quantize_q8_0(k).shape == (7, 3, 136)
        assert OPS.quantize_q8_0(k).dtype == torch.uint8
        # reference gather: [B, Hkv, Sk, row] in the cache dtypes
        kc = f((9, 16, 2, 136), torch.uint8)
        vc = f((9, 16, 2, 128), torch.float16)
        bt = f((3, 4), torch.int32)
        sl = f((3,), torch.int32)
        ko, vo = OPS.gather_paged_kv_q8(kc, vc, bt, sl, 64)
        assert ko.shape == (3, 2, 64, 136) and ko.dtype == torch.uint8
        assert vo.shape == (3, 2, 64, 128) and vo.dtype == torch.float16
        # contiguous forward: q [B, Hq, Sq, D] -> fp32 of that shape
        q = f((2, 8, 5, 128), torch.float32)
        kq = f((2, 2, 40, 136), torch.uint8)
        v = f((2, 2, 40, 128), torch.float16)
        o = OPS.forward(q, kq, v, 0.088)
        assert o.shape == (2, 8, 5, 128) and o.dtype == torch.float32
        # planar planes: paged attention and the Q8/Q8 gather
        cache = f((12, 2, 2, 2176), torch.uint8)
        qv = f((10, 8, 128), torch.bfloat16)
        qsl = f((4,), torch.int32)
        o = OPS.paged_attention(qv, cache[:, 0], cache[:, 1], bt, sl, qsl, 6, 64, 0.088, None)
        assert o.shape == (10, 8, 128) and o.dtype == torch.bfloat16
        o = OPS.paged_attention(qv, cache[:, 0], cache[:, 1], bt, sl, qsl, 6, 64, 0.088, None,
                                out_dtype=torch.float32)
        assert o.dtype == torch.float32
        k2, v2 = OPS.gather_paged_kv_q8q8(cache[:, 0], cache[:, 1], bt, sl, 32)
        assert k2.shape == v2.shape == (3, 2, 32, 136)
        q4 = f((3, 8, 2, 128), torch.float16)
        o = OPS.forward_paged_direct(q4, cache[:, 0], cache[:, 1], bt, sl, 0.088)
        assert o.shape == (3, 8, 2, 128) and o.dtype == torch.float32


def test_compile_fullgraph_keeps_ops_opaque():
    """A decode step written with the ops compiles as one graph: every op is
    a call_function node of its own (nothing traced into), the planes are
    views of one cache tensor.  The capturing backend returns outputs of the
    fake implementations' shapes without running anything."""
    graphs = []

    def capture(gm, example_inputs):
        graphs.append(gm)

        def run(*args):
            # the graph's outputs: the attention output of the step
            q = args[[n.name for n in gm.graph.find_nodes(op="placeholder")].index("l_query_")]
            return (torch.zeros(q.shape, dtype=torch.float32),)
        return run

    def step(query, key, value, slots, cache, block_table, seq_lens, qsl, ws, positions, cos_sin):
        kp, vp = cache[:, 0], cache[:, 1]
        torch.ops.gfx906_fa.rope_and_cache_q8_kv(positions, query, key, value, cos_sin, True, slots, kp, vp)
        return torch.ops.gfx906_fa.paged_attention(query, kp, vp, block_table, seq_lens, qsl, 1, 64, 0.088,
                                                   ws, out_dtype=torch.float32)

    B, Hq, Hkv = 3, 8, 2
    args = (torch.zeros(B, Hq, 128, dtype=torch.float16), torch.zeros(B, Hkv, 128, dtype=torch.float16),
            torch.zeros(B, Hkv, 128, dtype=torch.float16), torch.zeros(B, dtype=torch.int64),
            torch.zeros(8, 2, Hkv, 2176, dtype=torch.uint8), torch.zeros(B, 4, dtype=torch.int32),
            torch.ones(B, dtype=torch.int32), torch.arange(B + 1, dtype=torch.int32),
            torch.zeros(4096, dtype=torch.uint8), torch.zeros(B, dtype=torch.int64),
            torch.zeros(64, 128, dtype=torch.float16))
    torch._dynamo.reset()
    out = torch.compile(step, fullgraph=True, backend=capture)(*args)
    assert out.shape == (B, Hq, 128)
    assert len(graphs) == 1
    targets = [n.target for n in graphs[0].graph.nodes if n.op == "call_function"]
    assert torch.ops.gfx906_fa.rope_and_cache_q8_kv.default in targets or \
        torch.ops.gfx906_fa.rope_and_cache_q8_kv in targets
    assert torch.ops.gfx906_fa.paged_attention.default in targets or \
        torch.ops.gfx906_fa.paged_attention in targets
    torch._dynamo.reset()


def test_ops_reject_cpu_tensors():
    """The ops run the same checks as the functions: no CPU fallback."""
    import pytest
    with pytest.raises(RuntimeError, match="must be CUDA/HIP"):
        OPS.quantize_q8_0(torch.zeros(4, 128, dtype=torch.float16))
