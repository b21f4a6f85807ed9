"""GPU: prefill row tiles split over their keys.

A launch whose prefill row tiles (256 or 128 packed rows of one sequence and kv head)
are few and long - a prefix-cached chunk of tens to hundreds of tokens after a
long context, or a batch of such - has its row tiles cut into key ranges that
separate workgroups run; a combine kernel merges their partial (m, l, O).  The
shapes below make the device-side plan split: one row tile, several, a partial
last row tile, row tiles filling one to two rounds of workgroups cut to fill
one more, a batch mixing decode and prefill sequences, causal from key 0,
non-causal, a chunk inside its sequence (q_abs_offset), every query and
output dtype, and a HIP graph replayed with sequence lengths
that change the split.  Each case is checked against the oracle."""
import math

import numpy as np
import pytest
import torch

import gfx906_fa
import gfx906_fa_workloads as W
from gpu_common import announce, assert_close, batch_oracle, need_gpu, to_np_f32
from oracle import q8_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"

CASES = [
    # name, seq_lens, q_lens, Hq, Hkv
    ("chunk50_ctx4k", [4096 + 50], [50], 48, 8),            # 300 rows: a full and a partial row tile
    ("chunk12_x4_ctx8k", [8192 + 12] * 4, [12] * 4, 48, 8),  # 72 rows per sequence
    ("mixed_decode", [5000, 3000 + 100, 900, 70], [1, 100, 3, 70], 16, 2),
    ("gqa4_chunk200_ctx12k", [12000 + 200], [200], 32, 8),
    ("mqa_fresh2048", [2048], [2048], 8, 1),                 # causal from key 0, 64 row tiles
    ("two_rounds_16x100_ctx4k", [4096 + 100] * 16, [100] * 16, 48, 8),  # 48 row tiles: cut for 3 rounds
    # more than 1024 row tiles (the plan's per-item key-tile counts are then
    # recomputed instead of kept in LDS, and a capacity check runs): a fresh
    # 33000-token prefill (1032 row tiles at 8 rows per token) with a 40-token
    # chunk on a 100000-token context whose two row tiles exceed one CU's
    # share of the launch's key tiles and are cut
    ("many_tiles_33000_plus_chunk40_ctx100k", [33000, 100000 + 40], [33000, 40], 8, 1),
]


def _split_header(ws, b):
    """(work items, row tiles split over the keys) the call's plan kernel left
    in the workspace."""
    info = gfx906_fa.plan_info(b.num_seqs, b.num_tokens, b.Hq, b.Hkv, b.max_query_len, b.max_seq_len)
    off = info["pf_header_offset"]
    assert off >= 0, "the call has no prefill work list"
    hdr = ws[off:off + 8].view(torch.int32).cpu().tolist()
    return hdr[0], hdr[1]


def _sample(b, n=48, seed=0):
    """Query tokens to check: every sequence's first and last, plus a random set."""
    rng = np.random.default_rng(seed)
    qsl = b.qsl
    pick = set()
    for s in range(b.num_seqs):
        pick.update({int(qsl[s]), int(qsl[s + 1]) - 1})
    pick.update(rng.choice(b.num_tokens, min(n, b.num_tokens), replace=False).tolist())
    return sorted(pick)


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_split_prefill_matches_oracle(case):
    need_gpu()
    name, sls, qls, Hq, Hkv = case
    announce(f"prefill split {name}")
    b = W.build_batch(sls, qls, Hq, Hkv, seed=sum(map(ord, name)))
    ws = gfx906_fa.new_workspace(gfx906_fa.workspace_size(b.num_seqs, b.num_tokens, Hq, Hkv, b.max_query_len,
                                                          b.max_seq_len), DEV)
    out = W.attention(b, out_dtype=torch.float32, workspace=ws)
    torch.cuda.synchronize()
    items, nsplit = _split_header(ws, b)
    info = gfx906_fa.plan_info(b.num_seqs, b.num_tokens, Hq, Hkv, b.max_query_len, b.max_seq_len)
    dec_max, prow = info["dec_rows_max"], info["pf_rows"]
    tiles = sum(-(-q * (Hq // Hkv) // prow) for q in qls if q * (Hq // Hkv) > dec_max)
    # the plan split something: pieces beyond the row tiles, split row tiles listed
    assert nsplit > 0 and items > tiles, (items, nsplit, tiles)
    if name.startswith("many_tiles"):
        assert tiles > 1024
    rows = _sample(b) if b.num_tokens > 400 else None
    ref = batch_oracle(b, rows=rows)
    got = to_np_f32(out)
    if rows is not None:
        got, ref = got[rows], ref[rows]
    assert_close(got, ref)


@pytest.mark.parametrize("dt,extra", [(torch.float16, 2.0 ** -11), (torch.bfloat16, 2.0 ** -8)])
def test_split_prefill_output_dtypes(dt, extra):
    need_gpu()
    announce(f"prefill split out={dt}")
    b = W.build_batch([6000 + 40, 3000 + 90], [40, 90], 48, 8, seed=91)
    out = W.attention(b, out_dtype=dt)
    torch.cuda.synchronize()
    assert out.dtype == dt
    assert_close(to_np_f32(out), batch_oracle(b), extra=extra)


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_split_prefill_query_dtypes(dtype):
    """bf16 and fp32 models: the query read and the output written in the
    model dtype by the split pieces and the merge."""
    need_gpu()
    announce(f"prefill split query={dtype}")
    b = W.build_batch([5000 + 60], [60], 48, 8, dtype=dtype, seed=94)
    out = W.attention(b)
    torch.cuda.synchronize()
    assert out.dtype == b.query.dtype
    extra = {"bf16": 2.0 ** -8, "f32": 0.0}[dtype]
    assert_close(to_np_f32(out), batch_oracle(b), extra=extra)


def test_split_prefill_non_causal():
    """causal=0: every query row sees all seq_len keys (one-row oracle calls
    over the whole sequence)."""
    need_gpu()
    announce("prefill split non-causal")
    b = W.build_batch([3000, 5000], [60, 45], 48, 8, seed=92)
    kp, vp = b.planes()
    out = gfx906_fa.paged_attention(b.query, kp, vp, b.block_table, b.seq_lens_t, b.qsl_t, b.max_query_len,
                                    b.max_seq_len, b.scale, causal=False, out_dtype=torch.float32)
    torch.cuda.synchronize()
    kh, vh = O.planar_dequant(b.kv_cache.cpu().numpy())
    q = to_np_f32(b.query)
    ref = np.zeros(q.shape, np.float64)
    for s in range(b.num_seqs):
        for t in range(int(b.qsl[s]), int(b.qsl[s + 1])):
            ref[t] = O.paged_attention_ref(q[t:t + 1], kh, vh, b.block_table_np[s:s + 1],
                                           b.seq_lens[s:s + 1], np.array([0, 1], np.int32), b.scale)[0]
    assert_close(to_np_f32(out), ref)


def test_split_prefill_q_abs_offset():
    """q_abs_offset: a 40-token chunk at position 5000 of a 9000-token
    sequence.  The keys past the chunk exist but are masked; the plan cuts
    the 5040 visible keys only (one-row oracle calls up to each row's bound)."""
    need_gpu()
    announce("prefill split q_abs_offset")
    b = W.build_batch([9000], [40], 48, 8, seed=95)
    kp, vp = b.planes()
    qa = 5000
    out = gfx906_fa.paged_attention(b.query, kp, vp, b.block_table, b.seq_lens_t, b.qsl_t, b.max_query_len,
                                    b.max_seq_len, b.scale, out_dtype=torch.float32,
                                    q_abs_offset=torch.tensor([qa], dtype=torch.int32, device=DEV))
    torch.cuda.synchronize()
    kh, vh = O.planar_dequant(b.kv_cache.cpu().numpy())
    q = to_np_f32(b.query)
    ref = np.zeros(q.shape, np.float64)
    for t in range(b.num_tokens):
        ref[t] = O.paged_attention_ref(q[t:t + 1], kh, vh, b.block_table_np[0:1], np.array([qa + t + 1], np.int32),
                                       np.array([0, 1], np.int32), b.scale)[0]
    assert_close(to_np_f32(out), ref)


@pytest.mark.parametrize("nq", [60, 12])
def test_split_prefill_graph_replay(nq):
    """One chunked-prefill launch captured in a HIP graph, replayed with new
    sequence lengths (so a different split) and query values; every replay
    equals the eager call bit for bit, the last one the oracle.  60 tokens at
    48/8 are 360 rows per kv-head (256-row tiles), 12 tokens 72 rows (128-row
    key-interleaved tiles)."""
    need_gpu()
    announce(f"prefill split graph replay nq={nq}")
    B, Hq, Hkv, bs, max_blocks = 2, 48, 8, 16, 640
    assert gfx906_fa.plan_info(B, B * nq, Hq, Hkv, nq, max_blocks * bs)["pf_rows"] == (256 if nq == 60 else 128)
    NB = B * max_blocks
    T = B * nq
    rng = np.random.default_rng(93)
    cache = gfx906_fa.new_kv_cache(NB, bs, Hkv, device=DEV)
    kp, vp = cache[:, 0], cache[:, 1]
    allk = torch.from_numpy(rng.standard_normal((NB * bs, Hkv, 128)).astype(np.float16)).to(DEV)
    allv = torch.from_numpy(rng.standard_normal((NB * bs, Hkv, 128)).astype(np.float16)).to(DEV)
    gfx906_fa.reshape_and_cache_q8_kv(allk, allv, torch.arange(NB * bs, dtype=torch.int64, device=DEV), kp, vp)
    table = torch.from_numpy(rng.permutation(NB).astype(np.int32).reshape(B, max_blocks)).to(DEV)
    q = torch.empty((T, Hq, 128), dtype=torch.float16, device=DEV)
    sl = torch.empty(B, dtype=torch.int32, device=DEV)
    qsl = torch.arange(0, (B + 1) * nq, nq, dtype=torch.int32, device=DEV)
    out = torch.empty((T, Hq, 128), dtype=torch.float16, device=DEV)
    max_sl = max_blocks * bs
    ws = gfx906_fa.new_workspace(gfx906_fa.workspace_size(B, T, Hq, Hkv, nq, max_sl), DEV)
    scale = 1.0 / math.sqrt(128)

    def step(o):
        gfx906_fa.paged_attention(q, kp, vp, table, sl, qsl, nq, max_sl, scale, out=o, workspace=ws)

    def load(seed):
        r = np.random.default_rng(seed)
        sl.copy_(torch.from_numpy(r.integers(nq + 1000, max_sl + 1, B).astype(np.int32)))
        q.copy_(torch.from_numpy(r.standard_normal((T, Hq, 128)).astype(np.float16)))

    load(0)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step(out)  # warm-up off the capture
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step(out)
    eager = torch.empty_like(out)
    for seed in (1, 2, 3):
        load(seed)
        g.replay()
        torch.cuda.synchronize()
        step(eager)
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {seed} differs from eager"
    kh, vh = O.planar_dequant(cache.cpu().numpy())
    ref = O.paged_attention_ref(to_np_f32(q), kh, vh, table.cpu().numpy(), sl.cpu().numpy(),
                                qsl.cpu().numpy(), scale)
    assert_close(to_np_f32(out), ref, extra=2.0 ** -11)
