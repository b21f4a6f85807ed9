"""CPU: pin the oracle's cache write, gather, planar layout and attention.

Cache write: invariants of tests/test_quant.py:80-149 (written rows equal the
dense quantizer, untouched bytes stay, slot < 0 skips) plus the C
restatement.  Gather: a brute-force per-token loop is compared with a
vectorised fancy-index version written like tests/test_gather.py:15-38
(``_ref_gather``) and with the C restatement; edge cases seq_len = 0,
block_table = -1, Sk beyond the table.  Attention: float64 torch SDPA (math
path) on the same dequantized inputs, and closed-form cases."""
import math

import numpy as np
import pytest
import torch

from oracle import c_oracle as C
from oracle import q8_oracle as O


def test_reshape_and_cache_invariants():
    rng = np.random.default_rng(0)
    NB, bs, Hkv, D = 10, 16, 4, 128
    slots = np.array([5, 10, 20, 21, 22], np.int64)
    key = (rng.standard_normal((5, Hkv, D)) * 0.3).astype(np.float16)
    cache = np.zeros((NB, bs, Hkv, 136), np.uint8)
    O.reshape_and_cache_q8_aos(key, slots, cache)
    dense = O.quantize_q8_0_rows(key)
    for i, s in enumerate(slots):
        assert np.array_equal(cache[s // bs, s % bs], dense[i])
    mask = np.ones((NB, bs), bool)
    mask[slots // bs, slots % bs] = False
    assert not cache[mask].any()
    c2 = np.zeros_like(cache)
    C.reshape_and_cache(key, slots, c2)
    assert np.array_equal(cache, c2)


def test_reshape_and_cache_skip_negative_slot():
    rng = np.random.default_rng(1)
    key = rng.standard_normal((3, 2, 64)).astype(np.float16)
    cache = np.zeros((4, 16, 2, 68), np.uint8)
    O.reshape_and_cache_q8_aos(key, np.array([0, -1, 5]), cache)
    dense = O.quantize_q8_0_rows(key)
    assert np.array_equal(cache[0, 0], dense[0]) and np.array_equal(cache[0, 5], dense[2])
    cache[0, 0] = 0
    cache[0, 5] = 0
    assert not cache.any()


def _fancy_gather(kc, vc, bt, sl, Sk):
    """Vectorised form in the style of tests/test_gather.py:15-38, plus the
    table-bound rule of the v2 kernel (a logical block past the table or a
    -1 entry reads as invalid)."""
    B, M = bt.shape
    NB, bs, Hkv, _ = kc.shape
    t = np.arange(Sk)
    lb = t // bs
    pb = np.where(lb[None, :] < M, bt[:, np.minimum(lb, M - 1)], -1)      # [B, Sk]
    valid = (t[None, :] < sl[:, None]) & (pb >= 0)
    pbc = np.where(valid, pb, 0)
    k = kc[pbc, (t % bs)[None, :]]                                       # [B, Sk, Hkv, kb]
    v = vc[pbc, (t % bs)[None, :]]
    v = np.where(valid[..., None, None], v, 0)
    return np.transpose(k, (0, 2, 1, 3)), np.transpose(v, (0, 2, 1, 3)), valid


@pytest.mark.parametrize("vdt", ["f16", "q8"])
def test_gather_three_ways(vdt):
    rng = np.random.default_rng(2)
    NB, bs, Hkv, D = 8, 16, 2, 64
    kc = rng.integers(0, 256, (NB, bs, Hkv, 68), dtype=np.uint8)
    if vdt == "f16":
        vc = rng.standard_normal((NB, bs, Hkv, D)).astype(np.float16)
    else:
        vc = rng.integers(0, 256, (NB, bs, Hkv, 68), dtype=np.uint8)
    bt = rng.integers(0, NB, (4, 4)).astype(np.int32)
    bt[3, 2] = -1
    sl = np.array([0, 30, 64, 60], np.int32)
    Sk = 96  # beyond M * bs = 64: those tokens are invalid
    sentinel = np.full((4, Hkv, Sk, 68), 0xAB, np.uint8)
    k1, v1 = O.gather_paged_kv_q8_aos(kc, vc, bt, sl, Sk, k_out=sentinel.copy())
    k2, v2, valid = _fancy_gather(kc, vc, bt, sl, Sk)
    k3, v3 = C.gather(kc, vc, bt, sl, Sk, k_out=sentinel.copy())
    assert np.array_equal(v1, v2) and np.array_equal(v1, v3)
    assert np.array_equal(k1, k3)
    vb = np.transpose(valid[:, None, :].repeat(Hkv, 1), (0, 1, 2))
    assert np.array_equal(k1[vb], k2[vb])
    assert np.all(k1[~vb] == 0xAB)  # K untouched on invalid tokens


def test_planar_roundtrip_and_layout():
    rng = np.random.default_rng(3)
    bs, Hkv = 32, 3
    seq = 50
    k = rng.standard_normal((seq, Hkv, 128)).astype(np.float16)
    v = rng.standard_normal((seq, Hkv, 128)).astype(np.float16)
    bt = rng.permutation(6)[:2].astype(np.int32)
    pos = np.arange(seq)
    slots = bt[pos // bs].astype(np.int64) * bs + pos % bs
    cache = np.zeros(O.planar_cache_shape(6, bs, Hkv), np.uint8)
    O.planar_cache_write(k, v, slots, cache)
    ka, va = O.planar_to_aos(cache)
    kaos = np.zeros((6, bs, Hkv, 136), np.uint8)
    vaos = np.zeros_like(kaos)
    O.reshape_and_cache_q8_aos(k, slots, kaos)
    O.reshape_and_cache_q8_aos(v, slots, vaos)
    assert np.array_equal(ka, kaos) and np.array_equal(va, vaos)
    # positions are a bijection onto the 2048 int bytes of a sub-page
    tt, dd = np.meshgrid(np.arange(16), np.arange(128), indexing="ij")
    kp = O.planar_kpos(tt, dd).ravel()
    vp = O.planar_vpos(tt, dd).ravel()
    assert sorted(kp.tolist()) == list(range(2048)) and sorted(vp.tolist()) == list(range(2048))
    # V: the 4 tokens of a lane group are adjacent bytes for every d
    assert np.all(np.diff(O.planar_vpos(np.arange(4), 5)) == 1)
    # each 16-byte chunk of a lane's MFMA operand: K lane (t, g) reads
    # (4t+g)*16 and 1024 + (4t+g)*16 -> the 64 lanes cover each 1 KB half
    ko = sorted({int(O.planar_kpos(t, 8 * g)) // 16 for t in range(16) for g in range(4)})
    assert ko == list(range(64))


def _sdpa_ref(query, k_hat, v_hat, bt, sl, qsl, scale):
    """float64 torch SDPA (math backend) per sequence, GQA by repeat_interleave."""
    T, Hq, D = query.shape
    NB, bs, Hkv, _ = k_hat.shape
    out = torch.zeros((T, Hq, D), dtype=torch.float64)
    for s in range(len(sl)):
        q0, q1 = int(qsl[s]), int(qsl[s + 1])
        n, L = q1 - q0, int(sl[s])
        if n == 0 or L == 0:
            continue
        pos = np.arange(L)
        K = torch.from_numpy(k_hat[bt[s, pos // bs], pos % bs]).double()      # [L, Hkv, D]
        V = torch.from_numpy(v_hat[bt[s, pos // bs], pos % bs]).double()
        K = K.repeat_interleave(Hq // Hkv, dim=1).permute(1, 0, 2)
        V = V.repeat_interleave(Hq // Hkv, dim=1).permute(1, 0, 2)
        q = torch.from_numpy(query[q0:q1]).double().permute(1, 0, 2)
        mask = torch.arange(L)[None, :] <= (L - n + torch.arange(n))[:, None]
        o = torch.nn.functional.scaled_dot_product_attention(q[None], K[None], V[None],
                                                             attn_mask=mask[None, None], scale=scale)
        out[q0:q1] = o[0].permute(1, 0, 2)
    return out.numpy()


def _random_paged(rng, seq_lens, q_lens, Hq, Hkv, bs):
    bt, nb = O.make_block_table(rng, seq_lens, bs)
    k = rng.standard_normal((nb, bs, Hkv, 128)).astype(np.float16)
    v = rng.standard_normal((nb, bs, Hkv, 128)).astype(np.float16)
    kq = O.dequantize_q8_0_rows(O.quantize_q8_0_rows(k), 128)
    vq = O.dequantize_q8_0_rows(O.quantize_q8_0_rows(v), 128)
    qsl = np.concatenate([[0], np.cumsum(q_lens)]).astype(np.int32)
    q = rng.standard_normal((int(qsl[-1]), Hq, 128)).astype(np.float32)
    return q, kq, vq, bt, np.asarray(seq_lens, np.int32), qsl


def test_attention_oracle_matches_sdpa():
    rng = np.random.default_rng(4)
    q, kq, vq, bt, sl, qsl = _random_paged(rng, [37, 64, 5, 100], [1, 16, 5, 33], 12, 3, 16)
    scale = 1 / math.sqrt(128)
    a = O.paged_attention_ref(q, kq, vq, bt, sl, qsl, scale)
    b = _sdpa_ref(q, kq, vq, bt, sl, qsl, scale)
    assert np.max(np.abs(a - b)) < 1e-10


def test_attention_closed_forms():
    rng = np.random.default_rng(5)
    q, kq, vq, bt, sl, qsl = _random_paged(rng, [1, 20], [1, 20], 4, 2, 16)
    a = O.paged_attention_ref(q, kq, vq, bt, sl, qsl, 0.1)
    # single visible key: output = V row (GQA: q-head h reads kv-head h // 2)
    for h in range(4):
        assert np.allclose(a[0, h], vq[bt[0, 0], 0, h // 2])
        assert np.allclose(a[1, h], vq[bt[1, 0], 0, h // 2])  # first prefill row
    # zero query -> uniform scores -> mean of the visible V rows
    qz = np.zeros_like(q)
    az = O.paged_attention_ref(qz, kq, vq, bt, sl, qsl, 0.1)
    pos = np.arange(20)
    Vs = vq[bt[1, pos // 16], pos % 16]
    for j in range(20):
        assert np.allclose(az[1 + j, 3], Vs[: j + 1, 1].mean(0))


def test_attention_invariant_to_page_permutation():
    rng = np.random.default_rng(6)
    q, kq, vq, bt, sl, qsl = _random_paged(rng, [70], [3], 4, 1, 16)
    a = O.paged_attention_ref(q, kq, vq, bt, sl, qsl, 0.2)
    perm = rng.permutation(kq.shape[0])
    inv = np.argsort(perm)
    a2 = O.paged_attention_ref(q, kq[perm], vq[perm], inv[bt].astype(np.int32), sl, qsl, 0.2)
    assert np.allclose(a, a2, atol=1e-12)


def test_empty_rows_are_zero():
    rng = np.random.default_rng(7)
    q, kq, vq, bt, sl, qsl = _random_paged(rng, [16, 16], [1, 1], 2, 1, 16)
    sl = np.array([0, 16], np.int32)
    a = O.paged_attention_ref(q, kq, vq, bt, sl, qsl, 0.1)
    assert not a[0].any() and a[1].any()


def test_cpu_baseline_matches_oracle():
    """The timed CPU baseline (AoS gather + dequantize + fp32 SDPA) computes
    the same attention as the oracle, from the planar cache."""
    from oracle import cpu_baseline as CB
    rng = np.random.default_rng(8)
    bs, Hkv, Hq = 16, 2, 8
    seq_lens, q_lens = [40, 17, 64], [1, 3, 1]
    bt, nb = O.make_block_table(rng, seq_lens, bs)
    cache = np.zeros(O.planar_cache_shape(nb, bs, Hkv), np.uint8)
    k = rng.standard_normal((nb * bs, Hkv, 128)).astype(np.float16)
    v = rng.standard_normal((nb * bs, Hkv, 128)).astype(np.float16)
    O.planar_cache_write(k, v, np.arange(nb * bs, dtype=np.int64), cache)
    qsl = np.concatenate([[0], np.cumsum(q_lens)]).astype(np.int32)
    q = rng.standard_normal((int(qsl[-1]), Hq, 128)).astype(np.float32)
    ka, va = CB.aos_from_planar(cache)
    got = CB.attention_cpu(torch.from_numpy(q), ka, va, bt, np.asarray(seq_lens), np.asarray(q_lens), 0.09)
    kq, vq = O.planar_dequant(cache)
    exp = O.paged_attention_ref(q, kq, vq, bt, np.asarray(seq_lens, np.int32), qsl, 0.09)
    assert np.max(np.abs(got.numpy() - exp)) < 1e-4
    secs, tokens, nseq, passes, thr = CB.time_cpu_decode(torch.from_numpy(q), ka, va, bt, np.asarray(seq_lens),
                                                         np.asarray(q_lens), 0.09, budget_s=0.05)
    assert nseq >= 1 and tokens >= 40 and secs > 0


def test_cpu_prefill_baseline_matches_oracle():
    """The timed q-chunked CPU prefill (one kv-head's query heads, chunks of
    the prompt in spread order) computes the oracle's causal attention for
    those heads; the thread count is the process's CPU share."""
    import os
    from oracle import cpu_baseline as CB
    rng = np.random.default_rng(9)
    bs, Hkv, Hq, L = 16, 2, 6, 150
    bt, nb = O.make_block_table(rng, [L], bs)
    cache = np.zeros(O.planar_cache_shape(nb, bs, Hkv), np.uint8)
    k = rng.standard_normal((nb * bs, Hkv, 128)).astype(np.float16)
    v = rng.standard_normal((nb * bs, Hkv, 128)).astype(np.float16)
    O.planar_cache_write(k, v, np.arange(nb * bs, dtype=np.int64), cache)
    q = rng.standard_normal((L, Hq, 128)).astype(np.float32)
    ka, va = CB.aos_from_planar(cache)
    kq, vq = O.planar_dequant(cache)
    exp = O.paged_attention_ref(q, kq, vq, bt, np.array([L], np.int32), np.array([0, L], np.int32), 0.09)
    G = Hq // Hkv
    for h in range(Hkv):
        K, V = CB.head_kv_cpu(ka, va, bt[0], L, h)
        qh = torch.from_numpy(q[:, h * G:(h + 1) * G]).permute(1, 0, 2)
        got = torch.cat([CB.prefill_chunk_cpu(qh, K, V, r0, min(r0 + 64, L), L, 0.09) for r0 in range(0, L, 64)], 1)
        assert np.max(np.abs(got.permute(1, 0, 2).numpy() - exp[:, h * G:(h + 1) * G])) < 1e-4
    secs, flop, heads, done, nch, g, thr = CB.time_cpu_prefill(torch.from_numpy(q), ka, va, bt[0], L, 0.09,
                                                                chunk=64, budget_s=60.0)
    assert (heads, done, nch, g) == (Hkv, Hkv * 3, 3, G) and secs > 0
    assert flop == Hkv * 4.0 * 128 * G * (L * (L + 1) // 2)
    assert thr == CB.host_threads() <= len(os.sched_getaffinity(0))


def _flat_case(rng, B, Hq, Hkv, Sq, Skv):
    q = rng.standard_normal((B, Hq, Sq, 128)).astype(np.float32)
    k = rng.standard_normal((B, Hkv, Skv, 128)).astype(np.float16)
    v = rng.standard_normal((B, Hkv, Skv, 128)).astype(np.float16)
    return q, O.quantize_q8_0_rows(k), v


def test_flat_attention_oracle_matches_sdpa():
    rng = np.random.default_rng(9)
    q, kq, v = _flat_case(rng, 2, 6, 2, 5, 40)
    kv_max = np.array([40, 23], np.int32)
    qa = np.array([30, 3], np.int32)
    got = O.flat_attention_ref(q, kq, v, 0.1, kv_max=kv_max, q_abs_offset=qa)
    K = torch.from_numpy(O.dequantize_q8_0_rows(kq, 128)).double().repeat_interleave(3, dim=1)
    V = torch.from_numpy(v.astype(np.float64)).repeat_interleave(3, dim=1)
    pos = torch.arange(40)
    for b in range(2):
        mask = (pos[None, :] < int(kv_max[b])) & (pos[None, :] <= int(qa[b]) + torch.arange(5)[:, None])
        ref = torch.nn.functional.scaled_dot_product_attention(
            torch.from_numpy(q[b:b + 1]).double(), K[b:b + 1], V[b:b + 1], attn_mask=mask[None, None], scale=0.1)
        assert np.max(np.abs(got[b] - ref[0].numpy())) < 1e-10
    # single visible key -> that key's V row (batch 1, row 0 sees keys <= 3 ... cut by q_abs 3)
    one = O.flat_attention_ref(q, kq, v, 0.1, kv_max=np.array([1, 1], np.int32))
    assert np.allclose(one[0, 0, 0], v[0, 0, 0].astype(np.float64))
    assert np.allclose(one[1, 5, 4], v[1, 1, 0].astype(np.float64))


def test_flat_attention_oracle_matches_paged_oracle():
    """Same values as pages: flat (exact V = dequantized Q8 V) == paged oracle."""
    rng = np.random.default_rng(10)
    B, Hq, Hkv, Sq, Skv = 2, 4, 2, 3, 48
    q = rng.standard_normal((B, Hq, Sq, 128)).astype(np.float32)
    kq = O.quantize_q8_0_rows(rng.standard_normal((B, Hkv, Skv, 128)).astype(np.float16))
    vq = O.quantize_q8_0_rows(rng.standard_normal((B, Hkv, Skv, 128)).astype(np.float16))
    vh = O.dequantize_q8_0_rows(vq, 128)
    flat = O.flat_attention_ref(q, kq, vh, 0.08, q_abs_offset=np.full(B, Skv - Sq, np.int32))
    # pages of 16 tokens, sequence b owns pages b*3 .. b*3+2
    kh = O.dequantize_q8_0_rows(kq, 128)
    kpg = kh.transpose(0, 2, 1, 3).reshape(B * 3, 16, Hkv, 128)
    vpg = vh.transpose(0, 2, 1, 3).reshape(B * 3, 16, Hkv, 128)
    bt = np.arange(B * 3, dtype=np.int32).reshape(B, 3)
    paged = O.paged_attention_ref(q.transpose(0, 2, 1, 3).reshape(B * Sq, Hq, 128), kpg, vpg, bt,
                                  np.full(B, Skv, np.int32), np.arange(0, (B + 1) * Sq, Sq, dtype=np.int32), 0.08)
    assert np.max(np.abs(flat.transpose(0, 2, 1, 3).reshape(B * Sq, Hq, 128) - paged)) < 1e-12


def test_planar_v16_layout_bijection():
    tt, dd = np.meshgrid(np.arange(16), np.arange(128), indexing="ij")
    pos = O.planar_v16_pos(tt, dd).ravel()
    assert sorted(pos.tolist()) == list(range(0, 4096, 2))
    # a lane's 32 bytes: tokens 4T..4T+3 x d = i + 16(4hf + mm), mm = 0..3
    lane, hf = 21, 1
    T, i = lane // 16, lane % 16
    got = sorted(int(O.planar_v16_pos(4 * T + s, i + 16 * (4 * hf + mm))) for s in range(4) for mm in range(4))
    assert got == list(range(2048 * hf + 32 * lane, 2048 * hf + 32 * lane + 32, 2))


def test_flat_attention_oracle_mask():
    """An fp16 causal mask (0 / -inf) equals the inline causal bound; an
    additive mask matches SDPA with a float mask."""
    rng = np.random.default_rng(11)
    q, kq, v = _flat_case(rng, 2, 4, 2, 6, 30)
    qa = np.array([24, 10], np.int32)
    pos = np.arange(32)
    causal = np.where(pos[None, None, :] <= qa[:, None, None] + np.arange(6)[None, :, None], 0.0, -np.inf)
    a = O.flat_attention_ref(q, kq, v, 0.1, mask=causal.astype(np.float16))
    b = O.flat_attention_ref(q, kq, v, 0.1, q_abs_offset=qa)
    assert np.max(np.abs(a - b)) < 1e-12
    add = rng.standard_normal((2, 6, 32)).astype(np.float16)
    got = O.flat_attention_ref(q, kq, v, 0.1, mask=add)
    K = torch.from_numpy(O.dequantize_q8_0_rows(kq, 128)).double().repeat_interleave(2, dim=1)
    V = torch.from_numpy(v.astype(np.float64)).repeat_interleave(2, dim=1)
    ref = torch.nn.functional.scaled_dot_product_attention(
        torch.from_numpy(q).double(), K, V, attn_mask=torch.from_numpy(add[:, None, :, :30].astype(np.float64)),
        scale=0.1)
    assert np.max(np.abs(got - ref.numpy())) < 1e-10
