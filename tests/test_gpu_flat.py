"""GPU: the contiguous entry ``gfx906_fa.forward`` (the reference's
``extension/gfx906_fa.cpp:120-265``: AoS Q8_0 K, fp16 V) against
``oracle.flat_attention_ref``, and the repack kernels it uses, bit-exact."""
import numpy as np
import pytest
import torch

import gfx906_fa
from gpu_common import announce, assert_close, need_gpu
from oracle import q8_oracle as O

DEV = "cuda"
pytestmark = pytest.mark.gpu


def _inputs(seed, B, Hq, Hkv, Sq, Skv):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((B, Hq, Sq, 128)).astype(np.float32)
    k = rng.standard_normal((B, Hkv, Skv, 128)).astype(np.float16)
    v = rng.standard_normal((B, Hkv, Skv, 128)).astype(np.float16)
    return q, O.quantize_q8_0_rows(k), v


def test_pack_flat_kv_bitexact():
    need_gpu()
    announce("pack_flat_kv B=2 Hkv=3 Skv=37")
    B, Hkv, Skv = 2, 3, 37
    _, kq, v = _inputs(1, B, 3, Hkv, 1, Skv)
    skp = (Skv + 15) // 16
    kp = torch.full((B, Hkv, skp * 2176), 0xAB, dtype=torch.uint8, device=DEV)
    vp = torch.full((B, Hkv, skp * 4096), 0xAB, dtype=torch.uint8, device=DEV)
    L = gfx906_fa.lib()
    kd, vd = torch.from_numpy(kq).to(DEV), torch.from_numpy(v).to(DEV)  # alive across the launch
    err = L.gfx906_fa_amd_pack_flat_kv(gfx906_fa._ptr(kd), gfx906_fa._ptr(vd), gfx906_fa._ptr(kp),
                                      gfx906_fa._ptr(vp), B * Hkv, Skv, 128,
                                      gfx906_fa._stream(torch.device(DEV)))
    assert err == 0
    torch.cuda.synchronize()
    kp, vp = kp.cpu().numpy(), vp.cpu().numpy()
    qk, dk = O.unpack_q8_0_rows(kq, 128)
    dd = np.arange(128)
    vbits = v.view(np.uint16)
    for b in range(B):
        for h in range(Hkv):
            for t in range(skp * 16):
                sp, tt = divmod(t, 16)
                base = sp * 2176
                ints = kp[b, h, base + O.planar_kpos(tt, dd)].view(np.int8)
                sc = np.array([kp[b, h, base + O.planar_spos(0, tt, bb) + np.arange(2)] for bb in range(4)])
                vv = vp[b, h, sp * 4096 + O.planar_v16_pos(tt, dd)[:, None] + np.arange(2)].copy().view(np.uint16)[:, 0]
                if t < Skv:
                    assert np.array_equal(ints, qk[b, h, t])
                    assert np.array_equal(sc.copy().view("<f2").ravel(), dk[b, h, t])
                    assert np.array_equal(vv, vbits[b, h, t])
                else:  # padding tokens are zeros
                    assert not ints.any() and not sc.any() and not vv.any()


CASES = [
    # name, B, Hq, Hkv, Sq, Skv, kv_max, causal
    ("decode", 3, 8, 2, 1, 300, None, False),
    ("decode_kvmax", 3, 8, 2, 1, 300, [300, 17, 1], False),
    ("prefill_sq64_causal", 1, 8, 4, 64, 64, None, True),
    ("sweep_sq512", 1, 8, 4, 512, 1024, None, False),
    ("gqa_48_8_causal_ragged", 2, 48, 8, 100, 777, [777, 500], True),
]


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_forward_flat(case):
    need_gpu()
    name, B, Hq, Hkv, Sq, Skv, kv_max, causal = case
    announce(f"forward {name}")
    q, kq, v = _inputs(sum(map(ord, name)), B, Hq, Hkv, Sq, Skv)
    scale = 1.0 / np.sqrt(128)
    kvm = None if kv_max is None else np.asarray(kv_max, np.int32)
    qa = None
    if causal:  # the last Sq positions of each (possibly cut) sequence
        lens = np.full(B, Skv, np.int32) if kvm is None else kvm
        qa = (lens - Sq).astype(np.int32)
    out = gfx906_fa.forward(torch.from_numpy(q).to(DEV), torch.from_numpy(kq).to(DEV),
                            torch.from_numpy(v).to(DEV), scale,
                            kv_max=None if kvm is None else torch.from_numpy(kvm).to(DEV),
                            q_abs_offset=None if qa is None else torch.from_numpy(qa).to(DEV))
    torch.cuda.synchronize()
    assert out.shape == (B, Hq, Sq, 128) and out.dtype == torch.float32
    ref = O.flat_attention_ref(q, kq, v, scale, kv_max=kvm, q_abs_offset=qa)
    assert_close(out.cpu().numpy(), ref)


def test_forward_flat_rejects_bad_arguments():
    """The reference binding's checks (extension/gfx906_fa.cpp:131-227)."""
    need_gpu()
    q, kq, v = _inputs(3, 1, 2, 1, 4, 32)
    args = (torch.from_numpy(q).to(DEV), torch.from_numpy(kq).to(DEV), torch.from_numpy(v).to(DEV), 0.1)
    with pytest.raises(RuntimeError, match="mask must be fp16"):
        gfx906_fa.forward(*args, mask=torch.zeros((1, 4, 32), dtype=torch.float32, device=DEV))
    with pytest.raises(RuntimeError, match="mask.size"):
        gfx906_fa.forward(*args, mask=torch.zeros((1, 4, 16), dtype=torch.float16, device=DEV))
    with pytest.raises(RuntimeError, match="fp32"):
        gfx906_fa.forward(args[0].half(), *args[1:])
    with pytest.raises(RuntimeError, match="k_q8 last dim"):
        gfx906_fa.forward(args[0], args[1][..., :100].contiguous(), *args[2:])


def test_forward_flat_mask():
    """Materialised fp16 mask: a causal 0/-inf mask and a dense additive one
    (128 columns: four keys per load), and a dense one of 101 columns."""
    need_gpu()
    announce("forward mask B=2 Hq=8 Hkv=2 Sq=40 Skv=100")
    B, Hq, Hkv, Sq, Skv = 2, 8, 2, 40, 100
    q, kq, v = _inputs(77, B, Hq, Hkv, Sq, Skv)
    rng = np.random.default_rng(78)
    Skv_pad = 128
    pos = np.arange(Skv_pad)
    qa = np.array([60, 0], np.int32)
    causal = np.where(pos[None, None, :] <= qa[:, None, None] + np.arange(Sq)[None, :, None], 0.0, -np.inf)
    for m in (causal.astype(np.float16), rng.standard_normal((B, Sq, Skv_pad)).astype(np.float16)):
        out = gfx906_fa.forward(torch.from_numpy(q).to(DEV), torch.from_numpy(kq).to(DEV),
                                torch.from_numpy(v).to(DEV), 0.09, mask=torch.from_numpy(m).to(DEV))
        torch.cuda.synchronize()
        assert_close(out.cpu().numpy(), O.flat_attention_ref(q, kq, v, 0.09, mask=m))
    # 101 columns (more than Skv, not a multiple of 4): the mask is read one
    # element at a time instead of four keys per load
    m = rng.standard_normal((B, Sq, 101)).astype(np.float16)
    out = gfx906_fa.forward(torch.from_numpy(q).to(DEV), torch.from_numpy(kq).to(DEV),
                            torch.from_numpy(v).to(DEV), 0.09, mask=torch.from_numpy(m).to(DEV))
    torch.cuda.synchronize()
    assert_close(out.cpu().numpy(), O.flat_attention_ref(q, kq, v, 0.09, mask=m))
    with pytest.raises(RuntimeError, match="mutually exclusive"):
        gfx906_fa.forward(torch.from_numpy(q).to(DEV), torch.from_numpy(kq).to(DEV), torch.from_numpy(v).to(DEV),
                          0.09, mask=torch.from_numpy(m).to(DEV), q_abs_offset=torch.from_numpy(qa).to(DEV))


def test_forward_paged_direct_mask():
    """forward_paged_direct with a dense additive mask over the planar Q8 cache
    (the paged path's dequantized V) against the flat oracle on the same values."""
    need_gpu()
    announce("forward_paged_direct mask")
    B, Hq, Hkv, Sq, Skv, bs = 2, 6, 1, 20, 70, 16
    rng = np.random.default_rng(79)
    k = rng.standard_normal((B, Hkv, Skv, 128)).astype(np.float16)
    v = rng.standard_normal((B, Hkv, Skv, 128)).astype(np.float16)
    q = rng.standard_normal((B, Hq, Sq, 128)).astype(np.float32)
    nbs = (Skv + bs - 1) // bs
    bt = rng.permutation(B * nbs).astype(np.int32).reshape(B, nbs)
    cache = gfx906_fa.new_kv_cache(B * nbs, bs, Hkv, device=DEV)
    pos = np.arange(Skv)
    for b in range(B):
        slots = torch.from_numpy((bt[b, pos // bs].astype(np.int64) * bs + pos % bs)).to(DEV)
        gfx906_fa.reshape_and_cache_q8_kv(torch.from_numpy(k[b].transpose(1, 0, 2).copy()).to(DEV),
                                          torch.from_numpy(v[b].transpose(1, 0, 2).copy()).to(DEV),
                                          slots, cache[:, 0], cache[:, 1])
    m = rng.standard_normal((B, Sq, 80)).astype(np.float16)
    sl = np.array([70, 45], np.int32)
    out = gfx906_fa.forward_paged_direct(torch.from_numpy(q).to(DEV), cache[:, 0], cache[:, 1],
                                         torch.from_numpy(bt).to(DEV), torch.from_numpy(sl).to(DEV), 0.1,
                                         mask=torch.from_numpy(m).to(DEV))
    torch.cuda.synchronize()
    kq = O.quantize_q8_0_rows(k)
    vh = O.dequantize_q8_0_rows(O.quantize_q8_0_rows(v), 128)
    ref = O.flat_attention_ref(q, kq, vh, 0.1, kv_max=sl, mask=m)
    assert_close(out.cpu().numpy(), ref)
