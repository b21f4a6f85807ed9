"""GPU: KV caches larger than 4 GiB.

vLLM gives most of a GPU's memory to the KV cache (hundreds of GB on a
288 GB part), so page byte offsets beyond 2^32 are the normal case.  Each
test builds a small batch, copies its pages into a cache of more than
4.5 GiB at block ids whose byte offsets are past 4 GiB, shifts the block
table and slot mapping by the same number of blocks, and checks that every
entry point gives bit-identical bytes and outputs on the large cache and the
small one."""
import numpy as np
import pytest
import torch

import gfx906_fa
import gfx906_fa_workloads as W
from gpu_common import announce, need_gpu

pytestmark = pytest.mark.gpu
DEV = "cuda"
OFFSET_BYTES = 9 << 29  # 4.5 GiB: the relocated pages start past this offset


def _relocate(b):
    """(big cache, base block id, shifted block table, shifted slots)."""
    per_block = b.kv_cache[0].numel()
    base = -(-OFFSET_BYTES // per_block)
    big = torch.zeros((base + b.num_blocks,) + tuple(b.kv_cache.shape[1:]), dtype=torch.uint8, device=DEV)
    big[base:] = b.kv_cache
    assert base * per_block >= 1 << 32
    return big, base, (b.block_table + base).contiguous(), (b.slot_mapping + base * b.block_size).contiguous()


@pytest.mark.parametrize("bs", [16, 64])
def test_attention_and_gather_past_4gib(bs):
    need_gpu()
    announce(f"large cache attention bs={bs}")
    b = W.build_batch([5, 300, 1500, 700, 33, 4000], [1, 1, 5, 300, 33, 1], 12, 2, block_size=bs, seed=41)
    kp, vp = b.planes()
    big, base, bt, _ = _relocate(b)
    args = (b.seq_lens_t, b.qsl_t, b.max_query_len, b.max_seq_len, b.scale)
    out_s = gfx906_fa.paged_attention(b.query, kp, vp, b.block_table, *args, out_dtype=torch.float32)
    out_b = gfx906_fa.paged_attention(b.query, big[:, 0], big[:, 1], bt, *args, out_dtype=torch.float32)
    Sk = int(-(-b.max_seq_len // 32) * 32)
    gk_s, gv_s = gfx906_fa.gather_paged_kv_q8q8(kp, vp, b.block_table, b.seq_lens_t, Sk)
    gk_b, gv_b = gfx906_fa.gather_paged_kv_q8q8(big[:, 0], big[:, 1], bt, b.seq_lens_t, Sk)
    torch.cuda.synchronize()
    assert torch.equal(out_s, out_b)
    # K rows of invalid tokens are left as the buffers were allocated: compare valid rows
    sl = b.seq_lens
    for s in range(b.num_seqs):
        assert torch.equal(gk_s[s, :, :sl[s]], gk_b[s, :, :sl[s]])
    assert torch.equal(gv_s, gv_b)


def test_cache_writes_past_4gib():
    """The planar K+V write, the fused rotary + K/V write and the decode
    kernel's folded write land at the same bytes of the relocated pages."""
    need_gpu()
    announce("large cache writes")
    b = W.build_batch([70, 1000, 33], [1, 1, 1], 8, 2, seed=42, write_cache=False)
    kp, vp = b.planes()
    big, base, bt, slots = _relocate(b)
    # planar K+V write
    gfx906_fa.reshape_and_cache_q8_kv(b.key, b.value, b.slot_mapping, kp, vp)
    gfx906_fa.reshape_and_cache_q8_kv(b.key, b.value, slots, big[:, 0], big[:, 1])
    torch.cuda.synchronize()
    assert torch.equal(big[base:], b.kv_cache)
    # fused rotary + K/V write (rotates its query and key in place: copies)
    T = b.key.shape[0]
    pos = torch.arange(T, dtype=torch.int64, device=DEV)
    cs = W.rope_cos_sin_cache(T, 128, torch.float16, DEV)
    q1, k1 = torch.zeros(T, 8, 128, dtype=torch.float16, device=DEV), b.key.clone()
    q2, k2 = q1.clone(), b.key.clone()
    b.kv_cache.zero_()
    big.zero_()
    gfx906_fa.rope_and_cache_q8_kv(pos, q1, k1, b.value, cs, True, b.slot_mapping, kp, vp)
    gfx906_fa.rope_and_cache_q8_kv(pos, q2, k2, b.value, cs, True, slots, big[:, 0], big[:, 1])
    torch.cuda.synchronize()
    assert torch.equal(big[base:], b.kv_cache) and torch.equal(k1, k2)
    # decode with the step's cache write folded in: cache all but the last token
    # of each sequence, then the step writes it and attends
    starts = np.concatenate([[0], np.cumsum(b.seq_lens.astype(np.int64))])
    ctx = torch.from_numpy(np.concatenate([np.arange(starts[s], starts[s + 1] - 1)
                                           for s in range(b.num_seqs)])).to(DEV)
    new = torch.from_numpy(starts[1:] - 1).to(DEV)
    b.kv_cache.zero_()
    big.zero_()
    gfx906_fa.reshape_and_cache_q8_kv(b.key[ctx], b.value[ctx], b.slot_mapping[ctx], kp, vp)
    gfx906_fa.reshape_and_cache_q8_kv(b.key[ctx], b.value[ctx], slots[ctx], big[:, 0], big[:, 1])
    kn, vn = b.key[new].contiguous(), b.value[new].contiguous()
    args = (b.seq_lens_t, b.qsl_t, b.max_query_len, b.max_seq_len, b.scale)
    out_s = gfx906_fa.paged_attention(b.query, kp, vp, b.block_table, *args, out_dtype=torch.float32,
                                      new_key=kn, new_value=vn, slot_mapping=b.slot_mapping[new].contiguous())
    out_b = gfx906_fa.paged_attention(b.query, big[:, 0], big[:, 1], bt, *args, out_dtype=torch.float32,
                                      new_key=kn, new_value=vn, slot_mapping=slots[new].contiguous())
    torch.cuda.synchronize()
    assert torch.equal(big[base:], b.kv_cache)
    assert torch.equal(out_s, out_b)


def test_aos_cache_write_past_4gib():
    """The reference-layout AoS write (``reshape_and_cache_q8``, cache
    [NB, bs, Hkv, 136]) into block ids past 4 GiB."""
    need_gpu()
    announce("large AoS cache write")
    rng = np.random.default_rng(43)
    T, Hkv, bs = 300, 2, 16
    key = torch.from_numpy(rng.standard_normal((T, Hkv, 128), dtype=np.float32)).half().to(DEV)
    nb = T // bs + 2
    slots = torch.from_numpy(rng.permutation(nb * bs)[:T].astype(np.int64)).to(DEV)
    small = torch.zeros((nb, bs, Hkv, 136), dtype=torch.uint8, device=DEV)
    per_block = bs * Hkv * 136
    base = -(-OFFSET_BYTES // per_block)
    big = torch.zeros((base + nb, bs, Hkv, 136), dtype=torch.uint8, device=DEV)
    gfx906_fa.reshape_and_cache_q8(key, slots, small)
    gfx906_fa.reshape_and_cache_q8(key, slots + base * bs, big)
    torch.cuda.synchronize()
    assert base * per_block >= 1 << 32
    assert torch.equal(big[base:], small)
    assert int(big[:base].count_nonzero()) == 0
