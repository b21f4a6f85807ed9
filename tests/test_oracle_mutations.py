"""CPU: the oracle's pins catch plausible mistakes.

Each case plants one mistake in a copy of an oracle function (on the CPU,
never in the product) and shows that at least one of the independent checks
the oracle is pinned by rejects the mutant:
  quantizer  - the C restatement (oracle/q8_ref.c), the reference test's
               float64 oracle tolerance (tests/test_quant.py:29-52, 72-73),
               the known tie / extreme answers;
  attention  - float64 torch SDPA on the same dequantized inputs, the
               single-visible-key and uniform-score closed forms."""
import math

import numpy as np
import pytest
import torch

from oracle import c_oracle as C
from oracle import q8_oracle as O


# ---------------------------------------------------------------- quantizer
def _q_mutant(kind):
    def quant(x):
        xf = O._to_f32(x)
        D = xf.shape[-1]
        blk = xf.reshape(*xf.shape[:-1], D // 32, 32)
        with np.errstate(all="ignore"):
            amax = np.max(np.abs(blk), axis=-1)
            d = (amax / np.float32(127.0)).astype(np.float32)
            if kind == "id_from_fp16_d":          # 1/d taken from the stored fp16 scale
                d_for_id = d.astype(np.float16).astype(np.float32)
            else:
                d_for_id = d
            pos = d_for_id > 0
            idv = np.where(pos, np.float32(1.0) / np.where(pos, d_for_id, 1), 0).astype(np.float32)
            if kind == "divide_by_d":             # x / d instead of x * (1/d)
                prod = np.where(pos[..., None], blk / np.where(pos, d, 1)[..., None], 0).astype(np.float32)
            else:
                prod = (blk * idv[..., None]).astype(np.float32)
            if kind == "round_half_away":
                r = np.sign(prod) * np.floor(np.abs(prod) + 0.5)
            elif kind == "truncate":
                r = np.trunc(prod)
            else:
                r = np.rint(prod)
            q = np.clip(np.where(np.isnan(r), 0, r), -128, 127).astype(np.int8).reshape(xf.shape)
        dh = d.astype(np.float16)
        return O.pack_q8_0_rows(q, dh)
    return quant


def _q_checks(quant):
    """True when every pin accepts `quant`."""
    rng = np.random.default_rng(3)
    ok = True
    for dt, scale in [("f16", 1.0), ("f16", 37.0), ("bf16", 0.5), ("f32", 1e-3)]:
        x = (rng.standard_normal((257, 128)) * scale).astype(np.float32)
        x = x.astype(np.float16) if dt == "f16" else (O.f32_to_bf16_bits(x) if dt == "bf16" else x)
        ok &= np.array_equal(quant(x), C.quantize_rows(x))
    blk = np.zeros((1, 32), np.float32)
    blk[0, :8] = [127.0, -127.0, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5]
    q, _ = O.unpack_q8_0_rows(quant(blk.astype(np.float16)), 32)
    ok &= q[0, :8].tolist() == [127, -127, 0, 2, 2, 0, -2, -2]
    return bool(ok)


def test_quantizer_pins_accept_the_oracle():
    assert _q_checks(O.quantize_q8_0_rows)


@pytest.mark.parametrize("kind", ["id_from_fp16_d", "divide_by_d", "round_half_away", "truncate"])
def test_quantizer_pins_reject_mutant(kind):
    assert not _q_checks(_q_mutant(kind))


# ---------------------------------------------------------------- attention
def _case(seed=0):
    rng = np.random.default_rng(seed)
    seq_lens, q_lens, Hq, Hkv, bs = [37, 64, 5], [1, 16, 5], 12, 3, 16
    bt, nb = O.make_block_table(rng, seq_lens, bs)
    kq = O.dequantize_q8_0_rows(O.quantize_q8_0_rows(rng.standard_normal((nb, bs, Hkv, 128)).astype(np.float16)), 128)
    vq = O.dequantize_q8_0_rows(O.quantize_q8_0_rows(rng.standard_normal((nb, bs, Hkv, 128)).astype(np.float16)), 128)
    qsl = np.concatenate([[0], np.cumsum(q_lens)]).astype(np.int32)
    q = rng.standard_normal((int(qsl[-1]), Hq, 128)).astype(np.float32)
    return q, kq, vq, bt, np.asarray(seq_lens, np.int32), qsl


def _sdpa(q, kq, vq, bt, sl, qsl, scale):
    out = np.zeros(q.shape, np.float64)
    G = q.shape[1] // kq.shape[2]
    for s in range(len(sl)):
        q0, q1, L = int(qsl[s]), int(qsl[s + 1]), int(sl[s])
        pos = np.arange(L)
        K = torch.from_numpy(kq[bt[s, pos // 16], pos % 16]).double().repeat_interleave(G, 1).permute(1, 0, 2)
        V = torch.from_numpy(vq[bt[s, pos // 16], pos % 16]).double().repeat_interleave(G, 1).permute(1, 0, 2)
        qs = torch.from_numpy(q[q0:q1]).double().permute(1, 0, 2)
        m = torch.arange(L)[None, :] <= (L - (q1 - q0) + torch.arange(q1 - q0))[:, None]
        out[q0:q1] = torch.nn.functional.scaled_dot_product_attention(
            qs[None], K[None], V[None], attn_mask=m[None, None], scale=scale)[0].permute(1, 0, 2).numpy()
    return out


def _a_mutant(kind):
    def attn(q, kq, vq, bt, sl, qsl, scale):
        if kind == "gqa_modulo":        # kv-head h % Hkv instead of h // G
            Hq, Hkv = q.shape[1], kq.shape[2]
            perm = np.array([(h % Hkv) * (Hq // Hkv) + h // Hkv for h in range(Hq)])
            return O.paged_attention_ref(q[:, perm], kq, vq, bt, sl, qsl, scale)[:, np.argsort(perm)]
        if kind == "causal_off_by_one":  # row j sees keys < seq_len - n_q + j
            return O.paged_attention_ref(q, kq, vq, bt, sl - 1, qsl, scale)
        if kind == "missing_scale":
            return O.paged_attention_ref(q, kq, vq, bt, sl, qsl, 1.0)
        if kind == "k_v_swapped":
            return O.paged_attention_ref(q, vq, kq, bt, sl, qsl, scale)
        raise ValueError(kind)
    return attn


def _a_checks(attn):
    q, kq, vq, bt, sl, qsl = _case()
    scale = 1 / math.sqrt(128)
    ok = np.max(np.abs(attn(q, kq, vq, bt, sl, qsl, scale) - _sdpa(q, kq, vq, bt, sl, qsl, scale))) < 1e-9
    # closed form: a single visible key returns its V row (row 0 of a prefill)
    sl1 = np.array([1, 1, 1], np.int32)
    qsl1 = np.array([0, 1, 2, 3], np.int32)
    one = attn(q[:3], kq, vq, bt, sl1, qsl1, scale)
    G = q.shape[1] // kq.shape[2]
    for s in range(3):
        for h in range(q.shape[1]):
            ok &= np.allclose(one[s, h], vq[bt[s, 0], 0, h // G])
    return bool(ok)


def test_attention_pins_accept_the_oracle():
    assert _a_checks(O.paged_attention_ref)


@pytest.mark.parametrize("kind", ["gqa_modulo", "causal_off_by_one", "missing_scale", "k_v_swapped"])
def test_attention_pins_reject_mutant(kind):
    assert not _a_checks(_a_mutant(kind))
