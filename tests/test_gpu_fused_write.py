"""GPU: attention with the step's K/V cache write folded in
(``gfx906_fa_amd_paged_attention_kv_write``).

The fused call must leave the cache and the output bit-identical to the two
separate calls (``reshape_and_cache_q8_kv`` of the new tokens, then
``paged_attention``) on the same inputs.  Cases: decode (one new token),
speculative verify (five, possibly across a sub-page boundary), both decode
row classes in one batch, block sizes 16/32/64, skipped slots, long contexts
split over many workgroups, and the batches that take the write-first path
(prefill rows, an explicit q_abs_offset).  One case is also checked against
the oracle."""
import numpy as np
import pytest
import torch

import gfx906_fa
import gfx906_fa_workloads as W
from gpu_common import announce, assert_close, batch_oracle, need_gpu

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _step_inputs(seq_lens, q_lens, Hq, Hkv, bs=16, dtype="f16", seed=0, skip=()):
    """A batch whose cache holds every token except each sequence's last
    n_q (the step's new tokens), and those tokens' K/V rows and slots."""
    b = W.build_batch(seq_lens, q_lens, Hq, Hkv, block_size=bs, dtype=dtype, seed=seed, write_cache=False)
    starts = np.concatenate([[0], np.cumsum(b.seq_lens.astype(np.int64))])
    ctx, new = [], []
    for s, (sl, nq) in enumerate(zip(b.seq_lens, b.q_lens)):
        ctx.append(np.arange(starts[s], starts[s] + sl - nq))
        new.append(np.arange(starts[s] + sl - nq, starts[s] + sl))
    ctx = torch.from_numpy(np.concatenate(ctx)).to(DEV)
    new = torch.from_numpy(np.concatenate(new)).to(DEV)
    kp, vp = b.planes()
    gfx906_fa.reshape_and_cache_q8_kv(b.key[ctx], b.value[ctx], b.slot_mapping[ctx], kp, vp)
    slots = b.slot_mapping[new].clone()
    for t in skip:
        slots[t] = -1
    return b, b.key[new].contiguous(), b.value[new].contiguous(), slots


def _compare(b, k_new, v_new, slots, q_abs=None, odt=torch.float16):
    cache0 = b.kv_cache.clone()
    kp, vp = b.planes()
    args = (b.query, kp, vp, b.block_table, b.seq_lens_t, b.qsl_t, b.max_query_len, b.max_seq_len, b.scale)
    out_f = torch.empty((b.num_tokens, b.Hq, b.D), dtype=odt, device=DEV)
    gfx906_fa.paged_attention(*args, out=out_f, q_abs_offset=q_abs, new_key=k_new, new_value=v_new,
                              slot_mapping=slots)
    cache_f = b.kv_cache.clone()
    b.kv_cache.copy_(cache0)
    out_u = torch.empty_like(out_f)
    gfx906_fa.reshape_and_cache_q8_kv(k_new, v_new, slots, kp, vp)
    gfx906_fa.paged_attention(*args, out=out_u, q_abs_offset=q_abs)
    torch.cuda.synchronize()
    assert torch.equal(cache_f, b.kv_cache), "fused write left different cache bytes"
    assert torch.equal(out_f, out_u), "fused write changed the attention output"
    return out_f


@pytest.mark.parametrize("case", [
    ("decode", [1, 15, 16, 17, 300, 1000, 2049], [1] * 7, 48, 8, 16),
    ("decode-bs32", [5, 100, 1500, 33], [1] * 4, 12, 2, 32),
    ("decode-bs64", [64, 65, 700], [1] * 3, 8, 1, 64),
    ("verify", [3000, 5, 1200, 17, 18], [5] * 5, 6, 1, 16),          # 30 rows: two-row-group kernel
    ("verify-48", [3000, 20, 1200], [5] * 3, 48, 8, 16),
    ("two-classes", [900, 40, 33, 2000, 7], [1, 3, 1, 2, 3], 8, 1, 16),  # 8 and 24 rows
    ("long-split", [20000, 777, 12345], [1] * 3, 8, 1, 16),
    ("verify-36-rows", [3000, 6, 1200, 17, 20000], [6] * 5, 6, 1, 16),  # 36 rows: 48-row tiles
    ("verify-64-rows", [2500, 9, 4100], [8] * 3, 8, 1, 16),            # 64 rows: 32-row chunks
    ("three-classes", [30000, 800, 1200, 40], [5, 6, 1, 6], 6, 1, 16),  # 30, 36 and 6 rows
    ("verify-36-rows-short", [900, 6, 120], [6] * 3, 6, 1, 16),          # 36 rows: 32-row chunks
])
def test_fused_write_matches_separate_calls(case):
    need_gpu()
    name, sl, ql, hq, hkv, bs = case
    announce(f"fused kv write {name}")
    b, k_new, v_new, slots = _step_inputs(sl, ql, hq, hkv, bs=bs, seed=len(name))
    _compare(b, k_new, v_new, slots)


def test_fused_write_skipped_slots_and_bf16():
    need_gpu()
    announce("fused kv write skipped slots bf16")
    b, k_new, v_new, slots = _step_inputs([400, 37, 90, 1024], [1, 1, 5, 5], 12, 2, dtype="bf16", seed=3,
                                          skip=(1, 4, 9))
    _compare(b, k_new, v_new, slots, odt=torch.bfloat16)


@pytest.mark.parametrize("kind", ["prefill-rows", "q_abs"])
def test_fused_write_first_paths(kind):
    """Batches the decode kernels cannot fold the write into: the write runs
    first, with the same result as the separate calls."""
    need_gpu()
    announce(f"fused kv write fallback {kind}")
    if kind == "prefill-rows":
        b, k_new, v_new, slots = _step_inputs([64, 700, 1500, 33], [64, 200, 1, 1], 48, 8, seed=4)
        _compare(b, k_new, v_new, slots)
    else:
        b, k_new, v_new, slots = _step_inputs([100, 250], [1, 1], 8, 2, seed=5)
        qa = (b.seq_lens_t - 1).contiguous()
        _compare(b, k_new, v_new, slots, q_abs=qa)


def test_fused_write_full_cfg2_against_oracle_rows():
    """cfg2's shape (32 sequences, 2K-16K context, 48/8): fused equals
    separate, and sampled output rows match the oracle."""
    need_gpu()
    announce("fused kv write cfg2 shape")
    sl, ql, hq, hkv, dt = W.cfg_shape("cfg2")
    b, k_new, v_new, slots = _step_inputs(sl, ql, hq, hkv, dtype=dt, seed=0)
    out = _compare(b, k_new, v_new, slots, odt=torch.float32)
    rows = np.arange(0, b.num_tokens, 5)
    ref = batch_oracle(b, rows=rows)
    assert_close(out.cpu().numpy()[rows], ref[rows])


def test_fused_write_rejects_mismatched_dtype():
    need_gpu()
    announce("fused kv write dtype check")
    b, k_new, v_new, slots = _step_inputs([40, 50], [1, 1], 8, 2, seed=6)
    kp, vp = b.planes()
    with pytest.raises(RuntimeError):
        gfx906_fa.paged_attention(b.query, kp, vp, b.block_table, b.seq_lens_t, b.qsl_t, 1, 50, b.scale,
                                  new_key=k_new.float(), new_value=v_new.float(), slot_mapping=slots)
    with pytest.raises(RuntimeError):
        gfx906_fa.paged_attention(b.query, kp, vp, b.block_table, b.seq_lens_t, b.qsl_t, 1, 50, b.scale,
                                  new_key=k_new, new_value=v_new)
