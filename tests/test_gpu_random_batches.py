"""GPU: seeded random varlen batches against the float64 oracle.

Each case draws a batch the way a vLLM scheduler step can look: up to 100
sequences, each an empty query, a decode token, a short speculative-verify
block or a prefill chunk on a cached prefix, over a shuffled paged cache
with block sizes 16..64 and GQA shapes from 1 to 16 query heads per kv-head.
One call covers both decode row classes, the tiled prefill kernel (split
over the keys where its plan decides so) and the segment search on both
sides of 64 sequences.  The cases are fixed by their seeds; the tolerance is
the one in tests/test_gpu_attention.py (reference test strategy:
tests/test_fa_mixed_batch.py, tests/test_decode_batch.py)."""
import numpy as np
import pytest
import torch

import gfx906_fa
import gfx906_fa_workloads as W
from gpu_common import announce, assert_close, batch_oracle, need_gpu, to_np_f32

pytestmark = pytest.mark.gpu

HEADS = [(8, 1), (12, 2), (48, 8), (6, 1), (64, 4), (16, 16), (32, 8)]


def _draw(seed):
    rng = np.random.default_rng(1000 + seed)
    nseq = int(rng.choice([1, 3, 8, 31, 63, 64, 65, 100])) if seed % 3 else int(rng.integers(1, 101))
    hq, hkv = HEADS[seed % len(HEADS)]
    bs = int(rng.choice([16, 32, 64]))
    dt = "bf16" if seed % 2 else "f16"
    kind = rng.choice(4, size=nseq, p=[0.05, 0.55, 0.3, 0.1])
    ql = np.where(kind == 0, 0, np.where(kind == 1, 1, np.where(kind == 2, rng.integers(2, 7, nseq),
                                                                 rng.integers(7, 121, nseq))))
    ctx = rng.integers(0, 3000, nseq)
    sl = [int(q + c) if q + c > 0 else 1 for q, c in zip(ql, ctx)]
    return sl, [int(q) for q in ql], hq, hkv, bs, dt


@pytest.mark.parametrize("seed", range(24))
def test_random_batch_matches_oracle(seed):
    need_gpu()
    sl, ql, hq, hkv, bs, dt = _draw(seed)
    announce(f"random batch seed={seed} B={len(sl)} heads={hq}/{hkv} bs={bs} {dt} "
             f"max_q={max(ql)} max_k={max(sl)}")
    b = W.build_batch(sl, ql, hq, hkv, block_size=bs, dtype=dt, seed=2000 + seed)
    out = W.attention(b, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert_close(to_np_f32(out), batch_oracle(b))


def _draw_rows128(seed):
    """A batch whose prefill chunks have 65-128 rows per kv-head (the longest
    at least 65), beside decode and verify sequences: the 128-row
    key-interleaved prefill tiles, split or whole."""
    rng = np.random.default_rng(3000 + seed)
    hq, hkv = HEADS[seed % len(HEADS)]
    G = hq // hkv
    nseq = int(rng.integers(1, 41))
    lo, hi = 64 // G + 1, 128 // G
    kind = rng.choice(3, size=nseq, p=[0.5, 0.2, 0.3])
    ql = np.where(kind == 0, 1, np.where(kind == 1, rng.integers(2, max(3, lo), nseq), rng.integers(lo, hi + 1, nseq)))
    ql[int(rng.integers(nseq))] = int(rng.integers(lo, hi + 1))
    ctx = rng.integers(0, 20000, nseq)
    sl = [int(q + c) for q, c in zip(ql, ctx)]
    return sl, [int(q) for q in ql], hq, hkv, int(rng.choice([16, 32, 64])), "bf16" if seed % 2 else "f16"


@pytest.mark.parametrize("seed", range(12))
def test_random_batch_rows128_matches_oracle(seed):
    need_gpu()
    sl, ql, hq, hkv, bs, dt = _draw_rows128(seed)
    announce(f"random rows128 batch seed={seed} B={len(sl)} heads={hq}/{hkv} bs={bs} {dt} "
             f"max_q={max(ql)} max_k={max(sl)}")
    b = W.build_batch(sl, ql, hq, hkv, block_size=bs, dtype=dt, seed=4000 + seed)
    info = gfx906_fa.plan_info(b.num_seqs, b.num_tokens, hq, hkv, b.max_query_len, b.max_seq_len)
    assert info["pf_rows"] == 128, info
    out = W.attention(b, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert_close(to_np_f32(out), batch_oracle(b))


PROMPT_HEADS = [(8, 1), (64, 4), (24, 3), (48, 8), (32, 8), (16, 2)]


@pytest.mark.parametrize("seed", range(12))
def test_random_prompt_matches_oracle(seed):
    """A seeded prompt of 32 row tiles or more (so the plan writes the 64-key
    tile images and the prefill copies them into LDS), fresh or on a cached
    prefix, over block sizes 16..64 and six GQA shapes, against the float64
    oracle.  The worst error over such prompts sits in the first query rows,
    which see one or a few keys: there the output is V dequantized to fp16,
    off by at most half an fp16 ulp (1.95e-3 for |v| < 8)."""
    need_gpu()
    rng = np.random.default_rng(9000 + seed)
    hq, hkv = PROMPT_HEADS[seed % len(PROMPT_HEADS)]
    G = hq // hkv
    q = min(int(rng.integers(8192 // G + 1, 8192 // G + 900)), 2600)
    pre = int(rng.integers(1, 2500)) if seed % 3 == 2 else 0
    bs = int(rng.choice([16, 32, 64]))
    dt = "bf16" if seed % 2 else "f16"
    announce(f"random prompt seed={seed} heads={hq}/{hkv} bs={bs} {dt} q={q} prefix={pre}")
    b = W.build_batch([q + pre], [q], hq, hkv, block_size=bs, dtype=dt, seed=9100 + seed)
    info = gfx906_fa.plan_info(b.num_seqs, b.num_tokens, b.Hq, b.Hkv, b.max_query_len, b.max_seq_len)
    assert info["img_bytes"] > 0
    out = W.attention(b, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert_close(to_np_f32(out), batch_oracle(b))
