"""GPU: fused rotary embedding + Q8_0 K/V cache write, bit-exact.

The fused op (``gfx906_fa.rope_and_cache_q8_kv``) must leave query and key
exactly as the rotary-embedding restatement (``oracle.rope_ref``, vLLM's
semantics) does and write exactly the cache bytes of the planar K+V write of
the rotated key (``oracle.planar_cache_write``); it must also equal the
unfused GPU path (torch rotary in vLLM's native form, then
``reshape_and_cache_q8_kv``).  Cases: fp16 / bf16, neox and GPT-J pairs,
full and partial rotary dims, fp32 and model-dtype cos/sin tables, skipped
slots, out-of-range positions, views of a fused qkv tensor, and the
backend's do_rope_and_kv_cache_update on q8_0 pages followed by attention."""
import math

import numpy as np
import pytest
import torch

import gfx906_fa
from gpu_common import announce, assert_close, host_bits, need_gpu
from oracle import q8_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"
TD = {"f16": torch.float16, "bf16": torch.bfloat16}


def _dev(a, dt):
    a = np.asarray(a)
    if a.dtype == np.uint16:
        return torch.from_numpy(a.view(np.int16).copy()).view(torch.bfloat16).to(DEV)
    return torch.from_numpy(a.copy()).to(DEV)


def _case(dt, T, Hq, Hkv, rot, cs_dtype, seed, P=8192):
    rng = np.random.default_rng(seed)
    g = torch.Generator().manual_seed(seed)
    qkv = (torch.randn((T, Hq + 2 * Hkv, 128), generator=g) * 2.0).to(TD[dt]).to(DEV)
    cs = O.rope_cos_sin_cache(P, rot)
    if cs_dtype == "model":
        cs = O.f32_to_bf16_bits(cs) if dt == "bf16" else cs.astype(np.float16)
    pos = rng.integers(0, P, T).astype(np.int64)
    return qkv, _dev(cs, dt), cs, torch.from_numpy(pos).to(DEV), pos


@pytest.mark.parametrize("dt", ["f16", "bf16"])
@pytest.mark.parametrize("neox", [True, False])
@pytest.mark.parametrize("rot", [128, 64])
@pytest.mark.parametrize("cs_dtype", ["f32", "model"])
def test_rope_cache_write_bitexact(dt, neox, rot, cs_dtype):
    need_gpu()
    announce(f"rope+cache write {dt} neox={neox} rot={rot} cs={cs_dtype}")
    T, Hq, Hkv, bs, NB = 77, 8, 2, 16, 8
    qkv, cs_t, cs, pos_t, pos = _case(dt, T, Hq, Hkv, rot, cs_dtype, seed=rot + 2 * neox + (cs_dtype == "f32"))
    # signed zeros at angle 0 (sin = 0): x*cos - y*sin must keep IEEE zero signs
    qkv[:6, :, ::3] = -0.0
    qkv[:6, :, 1::7] = 0.0
    q, k, v = qkv[:, :Hq], qkv[:, Hq:Hq + Hkv], qkv[:, Hq + Hkv:]      # strided views
    q0, k0, v0 = host_bits(q.contiguous()), host_bits(k.contiguous()), host_bits(v.contiguous())
    pos[:6] = 0
    pos[[3, 40]] = [-5, cs.shape[0] + 7]                                 # out of range: unrotated
    pos_t = torch.from_numpy(pos).to(DEV)
    slots = np.random.default_rng(1).permutation(NB * bs)[:T].astype(np.int64)
    slots[[0, 11, 76]] = -1
    cache = torch.full((NB, 2, Hkv, bs // 16 * 2176), 0x77, dtype=torch.uint8, device=DEV)
    gfx906_fa.rope_and_cache_q8_kv(pos_t, q, k, v, cs_t, neox, torch.from_numpy(slots).to(DEV),
                                   cache[:, 0], cache[:, 1])
    torch.cuda.synchronize()
    qr, kr = O.rope_ref(q0, pos, cs, rot, neox), O.rope_ref(k0, pos, cs, rot, neox)
    assert np.array_equal(host_bits(q.contiguous()), qr)
    assert np.array_equal(host_bits(k.contiguous()), kr)
    assert np.array_equal(host_bits(v.contiguous()), v0)                 # value untouched
    exp = np.full(tuple(cache.shape), 0x77, np.uint8)
    O.planar_cache_write(kr, v0, slots, exp)
    assert np.array_equal(cache.cpu().numpy(), exp)


@pytest.mark.parametrize("heads", [(6, 1), (4, 4), (40, 8)])
def test_rope_head_counts(heads):
    """Head counts whose query and key rows share a 4-row iteration of a
    wave (6/1: rows 4, 5 query, 6 key), equal counts, and more than one
    32-row chunk per token."""
    need_gpu()
    Hq, Hkv = heads
    announce(f"rope heads {Hq}/{Hkv}")
    T, bs, NB = 45, 16, 4
    qkv, cs_t, cs, pos_t, pos = _case("f16", T, Hq, Hkv, 128, "model", seed=Hq * 7 + Hkv)
    q, k, v = qkv[:, :Hq], qkv[:, Hq:Hq + Hkv], qkv[:, Hq + Hkv:]
    q0, k0, v0 = host_bits(q.contiguous()), host_bits(k.contiguous()), host_bits(v.contiguous())
    slots = np.random.default_rng(3).permutation(NB * bs)[:T].astype(np.int64)
    cache = torch.zeros((NB, 2, Hkv, bs // 16 * 2176), dtype=torch.uint8, device=DEV)
    gfx906_fa.rope_and_cache_q8_kv(pos_t, q, k, v, cs_t, True, torch.from_numpy(slots).to(DEV),
                                   cache[:, 0], cache[:, 1])
    torch.cuda.synchronize()
    kr = O.rope_ref(k0, pos, cs, 128, True)
    assert np.array_equal(host_bits(q.contiguous()), O.rope_ref(q0, pos, cs, 128, True))
    assert np.array_equal(host_bits(k.contiguous()), kr)
    exp = np.zeros(tuple(cache.shape), np.uint8)
    O.planar_cache_write(kr, v0, slots, exp)
    assert np.array_equal(cache.cpu().numpy(), exp)


def _torch_rope_(x, positions, cos_sin, rot, neox):
    """vLLM's native rotary form with torch ops, written back into x."""
    cs = cos_sin[positions]
    cos, sin = cs.chunk(2, dim=-1)
    cos, sin = cos.unsqueeze(-2).to(x.dtype), sin.unsqueeze(-2).to(x.dtype)
    xr = x[..., :rot]
    if neox:
        x1, x2 = torch.chunk(xr, 2, dim=-1)
        o = torch.cat((x1 * cos - x2 * sin, x2 * cos + x1 * sin), dim=-1)
    else:
        x1, x2 = xr[..., ::2], xr[..., 1::2]
        o = torch.stack((x1 * cos - x2 * sin, x2 * cos + x1 * sin), dim=-1).flatten(-2)
    x[..., :rot] = o


@pytest.mark.parametrize("dt", ["f16", "bf16"])
@pytest.mark.parametrize("T", [5, 1500])
def test_fused_equals_unfused_path(dt, T):
    """Fused launch == torch rotary (vLLM native form, on the GPU) followed by
    the plain cache write, byte for byte; T = 1500 x 8 kv-heads takes the
    block-per-lane write kernel on the unfused side."""
    need_gpu()
    announce(f"rope fused vs unfused {dt} T={T}")
    Hq, Hkv, bs = 32, 8, 32
    NB = T // bs + 2
    qkv, cs_t, _, pos_t, _ = _case(dt, T, Hq, Hkv, 128, "model", seed=T)
    slots = torch.from_numpy(np.random.default_rng(2).permutation(NB * bs)[:T].astype(np.int64)).to(DEV)
    a = qkv.clone()
    c1 = torch.zeros((NB, 2, Hkv, bs // 16 * 2176), dtype=torch.uint8, device=DEV)
    c2 = torch.zeros_like(c1)
    gfx906_fa.rope_and_cache_q8_kv(pos_t, a[:, :Hq], a[:, Hq:Hq + Hkv], a[:, Hq + Hkv:], cs_t, True, slots,
                                   c1[:, 0], c1[:, 1])
    b = qkv.clone()
    _torch_rope_(b[:, :Hq], pos_t, cs_t, 128, True)
    _torch_rope_(b[:, Hq:Hq + Hkv], pos_t, cs_t, 128, True)
    gfx906_fa.reshape_and_cache_q8_kv(b[:, Hq:Hq + Hkv], b[:, Hq + Hkv:], slots, c2[:, 0], c2[:, 1])
    torch.cuda.synchronize()
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    assert torch.equal(c1, c2)


def test_rope_rejects_bad_arguments():
    need_gpu()
    announce("rope argument checks")
    qkv, cs_t, _, pos_t, _ = _case("f16", 4, 4, 1, 128, "model", seed=9)
    cache = gfx906_fa.new_kv_cache(2, 16, 1, device=DEV)
    slots = torch.arange(4, dtype=torch.int64, device=DEV)
    q, k, v = qkv[:, :4], qkv[:, 4:5], qkv[:, 5:6]
    with pytest.raises(RuntimeError):   # rot_dim not a multiple of 16 for neox
        gfx906_fa.rope_and_cache_q8_kv(pos_t, q, k, v, cs_t, True, slots, cache[:, 0], cache[:, 1], rot_dim=72)
    with pytest.raises(RuntimeError):   # int32 positions
        gfx906_fa.rope_and_cache_q8_kv(pos_t.int(), q, k, v, cs_t, True, slots, cache[:, 0], cache[:, 1])
    with pytest.raises(RuntimeError):   # fp32 rows
        gfx906_fa.rope_and_cache_q8_kv(pos_t, q.float(), k.float(), v.float(), cs_t, True, slots,
                                       cache[:, 0], cache[:, 1])


def test_backend_fused_rope_then_attention():
    """Gfx906FAImpl.do_rope_and_kv_cache_update on q8_0 pages for a prefill
    of 3 sequences, then forward: query / key rotated as the oracle does and
    the attention output within tolerance of the oracle over the rotated
    values."""
    need_gpu()
    announce("backend fused rope + forward")
    from gfx906_fa_backend import Gfx906FABackend, Gfx906FAImpl, Gfx906FAMetadata
    from gfx906_fa_paged import q8_planes
    Hq, Hkv, D, bs, NB = 12, 2, 128, 16, 24
    sl = [100, 37, 64]
    T = sum(sl)
    impl = Gfx906FAImpl(Hq, D, 1 / math.sqrt(D), Hkv, None, None, "q8_0")
    assert impl.fused_rope_kvcache_supported()
    kv = torch.zeros(Gfx906FABackend.get_kv_cache_page_size_bytes(bs, Hkv, D, "q8_0", torch.float16) * NB,
                     dtype=torch.uint8, device=DEV).view(Gfx906FABackend.get_kv_cache_shape(NB, bs, Hkv, D, "q8_0"))
    rng = np.random.default_rng(11)
    perm = rng.permutation(NB)
    nblk = [(n + bs - 1) // bs for n in sl]
    bt = np.full((3, max(nblk)), -1, np.int32)
    o = 0
    for s, n in enumerate(nblk):
        bt[s, :n] = perm[o:o + n]
        o += n
    positions = np.concatenate([np.arange(n) for n in sl]).astype(np.int64)
    slots = np.concatenate([O.slots_for(bt, s, np.arange(n), bs) for s, n in enumerate(sl)])
    g = torch.Generator().manual_seed(12)
    qkv = torch.randn((T, (Hq + 2 * Hkv) * D), generator=g).half().to(DEV)
    query, key, value = qkv[:, :Hq * D], qkv[:, Hq * D:(Hq + Hkv) * D], qkv[:, (Hq + Hkv) * D:]
    q0 = host_bits(query.contiguous()).reshape(T, Hq, D)
    k0 = host_bits(key.contiguous()).reshape(T, Hkv, D)
    cs_np = O.rope_cos_sin_cache(4096, D).astype(np.float16)
    cs = torch.from_numpy(cs_np).to(DEV)
    impl.do_rope_and_kv_cache_update(None, query, key, value, torch.from_numpy(positions).to(DEV), cs, True,
                                     kv, torch.from_numpy(slots).to(DEV))
    qsl = np.concatenate([[0], np.cumsum(sl)]).astype(np.int32)
    md = Gfx906FAMetadata(num_actual_tokens=T, max_query_len=max(sl), max_seq_len=max(sl),
                          query_start_loc=torch.from_numpy(qsl).to(DEV),
                          seq_lens=torch.tensor(sl, dtype=torch.int32, device=DEV),
                          block_table=torch.from_numpy(bt).to(DEV), slot_mapping=torch.from_numpy(slots).to(DEV))
    out = torch.empty((T, Hq * D), dtype=torch.float16, device=DEV)
    impl.forward(None, query.view(T, Hq, D), key.view(T, Hkv, D), value.view(T, Hkv, D), kv, md, output=out)
    torch.cuda.synchronize()
    qr = O.rope_ref(q0, positions, cs_np, D, True)
    assert np.array_equal(host_bits(query.contiguous()).reshape(T, Hq, D), qr)
    assert np.array_equal(host_bits(key.contiguous()).reshape(T, Hkv, D), O.rope_ref(k0, positions, cs_np, D, True))
    kp, vp = q8_planes(kv, Hkv, D)
    kh, vh = O.planar_dequant(torch.stack([kp, vp], 1).cpu().numpy())
    ref = O.paged_attention_ref(qr.astype(np.float32), kh, vh, bt, np.asarray(sl, np.int32), qsl, 1 / math.sqrt(D))
    assert_close(out.float().cpu().numpy().reshape(T, Hq, D), ref, extra=2.0 ** -11)
