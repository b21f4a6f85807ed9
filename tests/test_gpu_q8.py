"""GPU: Q8_0 quantize, cache writes and gathers are bit-exact.

Checked against the CPU oracle (oracle/q8_oracle.py), the committed golden
fixtures and, where built, the reference's own quant kernels compiled for
gfx950 from its sources (oracle/_ref).  Cases follow tests/test_quant.py and
tests/test_gather.py of the reference."""
import os

import numpy as np
import pytest
import torch

import gfx906_fa
from gpu_common import announce, host_bits, need_gpu, ref_lib, stream_ptr
from oracle import q8_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"
TD = {"f16": torch.float16, "bf16": torch.bfloat16, "f32": torch.float32}


def _rand(shape, dt, scale=1.0, seed=0):
    g = np.random.default_rng(seed)
    x = (g.standard_normal(shape) * scale).astype(np.float32)
    return torch.from_numpy(x).to(TD[dt]).to(DEV)


@pytest.mark.parametrize("dt", ["f16", "bf16", "f32"])
@pytest.mark.parametrize("shape", [(1, 32), (4, 128), (2, 8, 128), (1, 4, 64, 128), (4099, 128)])
def test_quantize_dense_bitexact(dt, shape):
    need_gpu()
    announce(f"quantize_q8_0 {dt} {shape}")
    for sc in (0.5, 1e-3, 300.0):
        x = _rand(shape, dt, sc, seed=len(shape))
        y = gfx906_fa.quantize_q8_0(x).cpu().numpy()
        assert np.array_equal(y, O.quantize_q8_0_rows(host_bits(x)))


def test_quantize_edge_fixture():
    need_gpu()
    announce("quantize_q8_0 edge fixture")
    g = np.load(os.path.join(os.path.dirname(__file__), "golden", "q8_edge.npz"))
    x = torch.from_numpy(g["f16"]).to(DEV)
    assert np.array_equal(gfx906_fa.quantize_q8_0(x).cpu().numpy(), g["f16_rows"])
    xb = torch.from_numpy(g["bf16_bits"].view(np.int16)).view(torch.bfloat16).to(DEV)
    assert np.array_equal(gfx906_fa.quantize_q8_0(xb).cpu().numpy(), g["bf16_rows"])


def test_quantize_matches_reference_kernel():
    need_gpu()
    L = ref_lib()
    if L is None:
        pytest.skip("oracle/_ref not built")
    announce("quantize_q8_0 vs reference kernel")
    x = _rand((65536, 128), "f16", 1.0, seed=9)
    x[:1024] *= 1e-3
    x[1024:2048] *= 100.0
    ours = gfx906_fa.quantize_q8_0(x)
    ref = torch.empty_like(ours)
    assert L.launch_quantize_q8_0_dense(x.data_ptr(), ref.data_ptr(), 65536, 128, stream_ptr()) == 0
    torch.cuda.synchronize()
    assert torch.equal(ours, ref)


def test_reshape_and_cache_q8():
    """tests/test_quant.py:80-117: slots [5,10,20,21,22], untouched slots stay 0."""
    need_gpu()
    announce("reshape_and_cache_q8 slots")
    NB, bs, Hkv, D = 10, 16, 4, 128
    slots = torch.tensor([5, 10, 20, 21, 22], dtype=torch.int64, device=DEV)
    key = _rand((5, Hkv, D), "f16", 0.3, seed=1)
    cache = torch.zeros((NB, bs, Hkv, 136), dtype=torch.uint8, device=DEV)
    gfx906_fa.reshape_and_cache_q8(key, slots, cache)
    exp = np.zeros((NB, bs, Hkv, 136), np.uint8)
    O.reshape_and_cache_q8_aos(host_bits(key), slots.cpu().numpy(), exp)
    assert np.array_equal(cache.cpu().numpy(), exp)
    L = ref_lib()
    if L is not None:
        c2 = torch.zeros_like(cache)
        assert L.launch_reshape_and_cache_q8(key.data_ptr(), slots.data_ptr(), c2.data_ptr(), 5, Hkv, D, bs,
                                             Hkv * D, D, bs * Hkv * 136, Hkv * 136, 136, stream_ptr()) == 0
        torch.cuda.synchronize()
        assert torch.equal(cache, c2)


def test_reshape_and_cache_q8_skip():
    """tests/test_quant.py:123-149: slot -1 skipped (D = 64)."""
    need_gpu()
    announce("reshape_and_cache_q8 skip")
    key = _rand((3, 2, 64), "f16", 1.0, seed=2)
    slots = torch.tensor([0, -1, 5], dtype=torch.int64, device=DEV)
    cache = torch.zeros((4, 16, 2, 68), dtype=torch.uint8, device=DEV)
    gfx906_fa.reshape_and_cache_q8(key, slots, cache)
    exp = np.zeros((4, 16, 2, 68), np.uint8)
    O.reshape_and_cache_q8_aos(host_bits(key), slots.cpu().numpy(), exp)
    assert np.array_equal(cache.cpu().numpy(), exp)


@pytest.mark.parametrize("dt", ["f16", "bf16"])
def test_reshape_and_cache_q8_strided(dt):
    """Non-contiguous key (a slice of a fused tensor) and a head-major cache
    viewed as [NB, bs, Hkv, bpr]: strides are honoured."""
    need_gpu()
    announce(f"reshape_and_cache_q8 strided {dt}")
    NB, bs, Hkv, D, T = 6, 16, 3, 128, 40
    fused = _rand((T, 3, Hkv, D), dt, 1.0, seed=3)
    key = fused[:, 1]
    phys = torch.full((NB, Hkv, bs, 136), 0x5A, dtype=torch.uint8, device=DEV)
    view = phys.permute(0, 2, 1, 3)
    slots = torch.from_numpy(np.random.default_rng(4).permutation(NB * bs)[:T].astype(np.int64)).to(DEV)
    slots[7] = -1
    gfx906_fa.reshape_and_cache_q8(key, slots, view)
    exp = np.full((NB, Hkv, bs, 136), 0x5A, np.uint8)
    O.reshape_and_cache_q8_aos(host_bits(key.contiguous()), slots.cpu().numpy(), exp.transpose(0, 2, 1, 3))
    assert np.array_equal(phys.cpu().numpy(), exp)


@pytest.mark.parametrize("dt", ["f16", "bf16", "f32"])
@pytest.mark.parametrize("bs", [16, 32])
def test_cache_write_kv_planar(dt, bs):
    need_gpu()
    announce(f"cache_write_kv planar {dt} bs={bs}")
    rng = np.random.default_rng(5)
    NB, Hkv, T = 9, 4, 100
    key = _rand((T, Hkv, 128), dt, 1.0, seed=6)
    val = _rand((T, Hkv, 128), dt, 3.0, seed=7)
    slots = rng.permutation(NB * bs)[:T].astype(np.int64)
    slots[[3, 50]] = -1
    cache = torch.full((NB, 2, Hkv, bs // 16 * 2176), 0xC3, dtype=torch.uint8, device=DEV)
    gfx906_fa.reshape_and_cache_q8_kv(key, val, torch.from_numpy(slots).to(DEV), cache[:, 0], cache[:, 1])
    exp = np.full(tuple(cache.shape), 0xC3, np.uint8)
    O.planar_cache_write(host_bits(key), host_bits(val), slots, exp)
    assert np.array_equal(cache.cpu().numpy(), exp)


@pytest.mark.parametrize("dt", ["f16", "bf16"])
@pytest.mark.parametrize("bs", [16, 32])
def test_cache_write_kv_planar_many_rows(dt, bs):
    """Above 4096 (token, kv-head) rows the write takes the block-per-lane
    kernel (one Q8_0 block per lane, 16 tokens per wave); a ragged last group
    of tokens and skipped slots included.  Bit-exact like the small path."""
    need_gpu()
    announce(f"cache_write_kv planar many rows {dt} bs={bs}")
    rng = np.random.default_rng(15)
    Hkv, T = 4, 1100            # 4400 rows; T % 16 = 12
    NB = (T + 40) // bs + 1
    key = _rand((T, Hkv, 128), dt, 1.0, seed=16)
    val = _rand((T, Hkv, 128), dt, 2.0, seed=17)
    slots = rng.permutation(NB * bs)[:T].astype(np.int64)
    slots[[0, 17, 1099]] = -1
    cache = torch.full((NB, 2, Hkv, bs // 16 * 2176), 0x3C, dtype=torch.uint8, device=DEV)
    gfx906_fa.reshape_and_cache_q8_kv(key, val, torch.from_numpy(slots).to(DEV), cache[:, 0], cache[:, 1])
    exp = np.full(tuple(cache.shape), 0x3C, np.uint8)
    O.planar_cache_write(host_bits(key), host_bits(val), slots, exp)
    assert np.array_equal(cache.cpu().numpy(), exp)


def test_cache_write_kv_strided_inputs():
    need_gpu()
    announce("cache_write_kv strided inputs")
    T, Hkv = 33, 2
    qkv = _rand((T, 2 + 2 * Hkv + 1, 128), "f16", 1.0, seed=8)
    key, val = qkv[:, 2:2 + Hkv], qkv[:, 2 + Hkv:2 + 2 * Hkv]
    slots = np.arange(T, dtype=np.int64) + 5
    cache = gfx906_fa.new_kv_cache(4, 16, Hkv, device=DEV)
    gfx906_fa.reshape_and_cache_q8_kv(key, val, torch.from_numpy(slots).to(DEV), cache[:, 0], cache[:, 1])
    exp = np.zeros(tuple(cache.shape), np.uint8)
    O.planar_cache_write(host_bits(key.contiguous()), host_bits(val.contiguous()), slots, exp)
    assert np.array_equal(cache.cpu().numpy(), exp)


def _gather_case(NB, bs, Hkv, D, bt, sl, Sk, vq8, seed):
    rng = np.random.default_rng(seed)
    kc = torch.from_numpy(rng.integers(0, 256, (NB, bs, Hkv, D // 32 * 34), dtype=np.uint8)).to(DEV)
    if vq8:
        vc = torch.from_numpy(rng.integers(0, 256, (NB, bs, Hkv, D // 32 * 34), dtype=np.uint8)).to(DEV)
    else:
        vc = torch.from_numpy(rng.standard_normal((NB, bs, Hkv, D)).astype(np.float16)).to(DEV)
    btt = torch.from_numpy(np.asarray(bt, np.int32)).to(DEV)
    slt = torch.from_numpy(np.asarray(sl, np.int32)).to(DEV)
    B = btt.shape[0]
    kbuf = torch.full((B, Hkv, Sk, D // 32 * 34), 0xAB, dtype=torch.uint8, device=DEV)
    ko, vo = gfx906_fa.gather_paged_kv_q8(kc, vc, btt, slt, Sk, k_out=kbuf)
    assert ko is kbuf
    ke, ve = O.gather_paged_kv_q8_aos(kc.cpu().numpy(), vc.cpu().numpy(), np.asarray(bt, np.int32),
                                      np.asarray(sl), Sk, k_out=np.full(tuple(kbuf.shape), 0xAB, np.uint8))
    assert np.array_equal(ko.cpu().numpy(), ke)
    assert np.array_equal(vo.cpu().numpy(), ve)


@pytest.mark.parametrize("vq8", [False, True])
def test_gather_basic(vq8):
    """tests/test_gather.py:41-87: seq_lens [0, 30, Sk], random table."""
    need_gpu()
    announce(f"gather basic vq8={vq8}")
    rng = np.random.default_rng(0)
    bt = rng.integers(0, 8, (3, 4))
    _gather_case(8, 16, 2, 64, bt, [0, 30, 64], 64, vq8, 1)


@pytest.mark.parametrize("vq8", [False, True])
def test_gather_stress_and_edges(vq8):
    """tests/test_gather.py:90-128 plus -1 pages and Sk past the table."""
    need_gpu()
    announce(f"gather stress vq8={vq8}")
    rng = np.random.default_rng(42)
    bt = rng.integers(0, 64, (8, 8))
    bt[2, 3] = -1
    sl = rng.integers(1, 129, 8)
    sl[5] = 0
    _gather_case(64, 16, 4, 128, bt, sl, 128, vq8, 2)
    _gather_case(64, 16, 4, 128, bt, np.minimum(sl + 60, 200), 192, vq8, 3)  # Sk > M*bs


@pytest.mark.parametrize("bs", [8, 32])
@pytest.mark.parametrize("vq8", [False, True])
def test_gather_block_sizes(vq8, bs):
    """Both word paths of the row gather: block_size 8 takes the per-word
    kernel (8-byte words), 32 the 16-byte slab kernel (a 16-token slab inside
    one page); seq_lens that end mid-slab on odd token counts (an 8-byte K
    tail), -1 pages, seq_len 0."""
    need_gpu()
    announce(f"gather block_size={bs} vq8={vq8}")
    rng = np.random.default_rng(7 + bs)
    M = 256 // bs
    bt = rng.integers(0, 40, (6, M))
    bt[4, 1] = -1
    sl = np.array([0, 17, 255, 33, 200, 129])
    _gather_case(40, bs, 3, 128, bt, sl, 256, vq8, 4)


@pytest.mark.parametrize("bs", [16, 64])
def test_gather_planar(bs):
    need_gpu()
    announce(f"gather planar bs={bs}")
    rng = np.random.default_rng(11)
    NB, Hkv, B = 12, 3, 4
    M = 3
    bt = rng.integers(0, NB, (B, M)).astype(np.int32)
    bt[1, 2] = -1
    sl = np.array([0, 3 * bs, bs + 7, 2 * bs], np.int32)
    Sk = ((M * bs + 16 + 31) // 32) * 32
    cache = torch.from_numpy(rng.integers(0, 256, (NB, 2, Hkv, bs // 16 * 2176), dtype=np.uint8)).to(DEV)
    kbuf = torch.full((B, Hkv, Sk, 136), 0xAB, dtype=torch.uint8, device=DEV)
    ko, vo = gfx906_fa.gather_paged_kv_q8q8(cache[:, 0], cache[:, 1], torch.from_numpy(bt).to(DEV),
                                            torch.from_numpy(sl).to(DEV), Sk, k_out=kbuf)
    ka, va = O.planar_to_aos(cache.cpu().numpy())
    ke, ve = O.gather_paged_kv_q8_aos(ka, va, bt, sl, Sk, k_out=np.full(tuple(kbuf.shape), 0xAB, np.uint8))
    assert np.array_equal(ko.cpu().numpy(), ke)
    assert np.array_equal(vo.cpu().numpy(), ve)


def test_gather_planar_unaligned_outputs():
    """The planar gather's per-word kernel, taken for outputs that are not
    16-byte aligned (here 4 bytes past an allocation), through the C ABI."""
    need_gpu()
    announce("gather planar unaligned outputs")
    rng = np.random.default_rng(12)
    NB, Hkv, B, M, bs = 10, 2, 3, 2, 32
    bt = rng.integers(0, NB, (B, M)).astype(np.int32)
    bt[2, 1] = -1
    sl = np.array([5, 64, 40], np.int32)
    Sk = 64
    cache = torch.from_numpy(rng.integers(0, 256, (NB, 2, Hkv, bs // 16 * 2176), dtype=np.uint8)).to(DEV)
    n = B * Hkv * Sk * 136
    kraw = torch.full((n + 4,), 0xAB, dtype=torch.uint8, device=DEV)
    vraw = torch.full((n + 4,), 0xCD, dtype=torch.uint8, device=DEV)
    btt, slt = torch.from_numpy(bt).to(DEV), torch.from_numpy(sl).to(DEV)
    kp, vp = cache[:, 0], cache[:, 1]
    err = gfx906_fa.lib().gfx906_fa_amd_gather_planar(
        kp.data_ptr(), vp.data_ptr(), btt.data_ptr(), slt.data_ptr(), kraw.data_ptr() + 4, vraw.data_ptr() + 4,
        B, Hkv, Sk, 128, bs, M, kp.stride(0), kp.stride(1), stream_ptr())
    assert err == 0
    torch.cuda.synchronize()
    ka, va = O.planar_to_aos(cache.cpu().numpy())
    ke, ve = O.gather_paged_kv_q8_aos(ka, va, bt, sl, Sk, k_out=np.full((B, Hkv, Sk, 136), 0xAB, np.uint8))
    assert np.array_equal(kraw[4:].cpu().numpy().reshape(B, Hkv, Sk, 136), ke)
    assert np.array_equal(vraw[4:].cpu().numpy().reshape(B, Hkv, Sk, 136), ve)
    assert int(kraw[:4].sum()) == 4 * 0xAB and int(vraw[:4].sum()) == 4 * 0xCD


def test_roundtrip_write_gather_dequant():
    """tests/test_q8_roundtrip.py: write -> gather -> dequant equals dense
    quantize -> dequant, for K and V."""
    need_gpu()
    announce("roundtrip write/gather/dequant")
    T, Hkv, bs = 128, 8, 16
    key = _rand((T, Hkv, 128), "f16", 0.5, seed=12)
    val = _rand((T, Hkv, 128), "f16", 0.5, seed=13)
    bt = torch.arange(T // bs, dtype=torch.int32, device=DEV).view(1, -1)
    pos = torch.arange(T, device=DEV)
    slots = (bt[0, pos // bs].long() * bs + pos % bs)
    cache = gfx906_fa.new_kv_cache(16, bs, Hkv, device=DEV)
    gfx906_fa.reshape_and_cache_q8_kv(key, val, slots, cache[:, 0], cache[:, 1])
    ko, vo = gfx906_fa.gather_paged_kv_q8q8(cache[:, 0], cache[:, 1], bt,
                                            torch.tensor([T], dtype=torch.int32, device=DEV), T)
    for src, got in ((key, ko), (val, vo)):
        rec = O.dequantize_q8_0_rows(got[0].permute(1, 0, 2).cpu().numpy(), 128)
        ref = O.dequantize_q8_0_rows(gfx906_fa.quantize_q8_0(src).cpu().numpy(), 128)
        assert np.array_equal(rec, ref)


def _ref_abi():
    """This library's reference-named launchers, with their reference
    signatures (extension/gfx906_fa.cpp:38-115)."""
    return gfx906_fa.lib()


def test_reference_named_quantize_and_cache_write():
    """launch_quantize_q8_0_dense and launch_reshape_and_cache_q8 of THIS
    library, called as the reference's binding calls them
    (extension/gfx906_fa.cpp:273-374): fp16 input, key strides in elements,
    cache strides in bytes, slot < 0 skipped - byte for byte against the
    oracle."""
    need_gpu()
    L = _ref_abi()
    announce("reference ABI: launch_quantize_q8_0_dense")
    x = _rand((777, 128), "f16", 1.0, seed=40)
    x[:100] *= 1e-3
    y = torch.full((777, 136), 0xCD, dtype=torch.uint8, device=DEV)
    assert L.launch_quantize_q8_0_dense(x.data_ptr(), y.data_ptr(), 777, 128, stream_ptr()) == 0
    torch.cuda.synchronize()
    assert np.array_equal(y.cpu().numpy(), O.quantize_q8_0_rows(host_bits(x)))
    x64 = _rand((33, 64), "f16", 3.0, seed=41)   # D = 64: two blocks per row
    y64 = torch.empty((33, 68), dtype=torch.uint8, device=DEV)
    assert L.launch_quantize_q8_0_dense(x64.data_ptr(), y64.data_ptr(), 33, 64, stream_ptr()) == 0
    torch.cuda.synchronize()
    assert np.array_equal(y64.cpu().numpy(), O.quantize_q8_0_rows(host_bits(x64)))

    announce("reference ABI: launch_reshape_and_cache_q8")
    NB, bs, Hkv, D, T = 7, 16, 4, 128, 50
    fused = _rand((T, 3, Hkv, D), "f16", 1.0, seed=42)
    key = fused[:, 1]                                   # token stride 3*Hkv*D elements
    rng = np.random.default_rng(43)
    slots = rng.permutation(NB * bs)[:T].astype(np.int64)
    slots[[3, 17]] = -1
    sl_t = torch.from_numpy(slots).to(DEV)
    cache = torch.full((NB, bs, Hkv, 136), 0x5A, dtype=torch.uint8, device=DEV)
    err = L.launch_reshape_and_cache_q8(key.data_ptr(), sl_t.data_ptr(), cache.data_ptr(), T, Hkv, D, bs,
                                        key.stride(0), key.stride(1), cache.stride(0), cache.stride(1),
                                        cache.stride(2), stream_ptr())
    assert err == 0
    torch.cuda.synchronize()
    exp = np.full((NB, bs, Hkv, 136), 0x5A, np.uint8)
    O.reshape_and_cache_q8_aos(host_bits(key.contiguous()), slots, exp)
    assert np.array_equal(cache.cpu().numpy(), exp)


@pytest.mark.parametrize("v_row_elems", [128, 160, 130])
def test_reference_named_gather(v_row_elems):
    """launch_gather_paged_kv_q8 of THIS library with the reference's
    conventions (extension/gfx906_fa_gather.cu:362-425): K cache strides in
    bytes, V cache strides in fp16 elements (converted to bytes inside).  V
    rows padded to 160 or 130 elements make the element strides differ from
    the byte strides (130 also leaves rows only 4-byte aligned).  Against
    the oracle's v2 contract: V zeroed and K untouched on invalid tokens,
    -1 pages, seq_len 0, Sk past the table."""
    need_gpu()
    L = _ref_abi()
    announce(f"reference ABI: launch_gather_paged_kv_q8 v_row={v_row_elems}")
    rng = np.random.default_rng(44)
    NB, bs, Hkv, D, B, M = 40, 16, 3, 128, 5, 6
    kc = torch.from_numpy(rng.integers(0, 256, (NB, bs, Hkv, 136), dtype=np.uint8)).to(DEV)
    vfull = torch.from_numpy(rng.standard_normal((NB, bs, Hkv, v_row_elems)).astype(np.float16)).to(DEV)
    vc = vfull[..., :D]
    bt = rng.integers(0, NB, (B, M)).astype(np.int32)
    bt[1, 4] = -1
    sl = np.array([0, 90, 17, M * bs, 33], np.int32)
    Sk = ((M * bs + 20 + 31) // 32) * 32               # past the table
    btt, slt = torch.from_numpy(bt).to(DEV), torch.from_numpy(sl).to(DEV)
    ko = torch.full((B, Hkv, Sk, 136), 0xAB, dtype=torch.uint8, device=DEV)
    vo = torch.full((B, Hkv, Sk, D), 7.0, dtype=torch.float16, device=DEV)
    err = L.launch_gather_paged_kv_q8(kc.data_ptr(), vc.data_ptr(), btt.data_ptr(), slt.data_ptr(), ko.data_ptr(),
                                      vo.data_ptr(), B, Hkv, Sk, D, 136, bs, M, kc.stride(0), kc.stride(1),
                                      kc.stride(2), vc.stride(0), vc.stride(1), vc.stride(2), stream_ptr())
    assert err == 0
    torch.cuda.synchronize()
    ke, ve = O.gather_paged_kv_q8_aos(kc.cpu().numpy(), vc.contiguous().cpu().numpy(), bt, sl, Sk,
                                      k_out=np.full((B, Hkv, Sk, 136), 0xAB, np.uint8))
    assert np.array_equal(ko.cpu().numpy(), ke)
    assert np.array_equal(vo.cpu().numpy(), ve)
