"""GPU: prefill sequences of 65-384 packed rows per kv-head.

Sequences whose query rows (n_q * G per kv-head) fill at most half of a
256-row tile run on 128-row key-interleaved tiles (KS = 2): two consumer
groups take alternate 64-key tiles for the same rows and merge their partial
states at the end.  The host plan chooses them when the longest prefill
sequence has at most 128 rows per kv-head; more rows keep the 256-row tile.
Each case asserts the tile size the plan chose (plan_info ``pf_rows``) and
checks the output against the oracle: rows per kv-head 65, 72, 96, 128, 192,
255, 300 and 384, alone, several per batch, mixed with decode rows, split
over the keys and whole, with 1, 2 and 3 key tiles (both groups' padding
paths), every output dtype, and a chunk inside its sequence
(q_abs_offset)."""
import numpy as np
import pytest
import torch

import gfx906_fa
import gfx906_fa_workloads as W
from gpu_common import announce, assert_close, batch_oracle, need_gpu, to_np_f32

pytestmark = pytest.mark.gpu
DEV = "cuda"

CASES = [
    # name, seq_lens, q_lens, Hq, Hkv, rows per tile the plan must choose
    ("rows65_g5_ctx6k", [6000 + 13], [13], 40, 8, 128),
    ("rows72_x8_ctx8k", [8192 + 12] * 8, [12] * 8, 48, 8, 128),
    ("rows96_g8_ctx5k", [5000 + 12, 4100 + 12], [12, 12], 64, 8, 128),
    ("rows128_g8_ctx9k", [9000 + 16], [16], 64, 8, 128),
    ("rows192_g6_ctx7k", [7000 + 32], [32], 48, 8, 256),
    ("rows255_g5_ctx3k", [3000 + 51], [51], 40, 8, 256),
    ("rows300_g6_ctx12k", [12000 + 50], [50], 48, 8, 256),
    ("rows384_g8_ctx4k", [4000 + 48, 2500 + 48], [48, 48], 64, 8, 256),
    # decode sequences (16- and 32-row classes) next to 72-row chunks
    ("mixed_decode_rows72", [7000, 3000 + 12, 900, 5000 + 5, 12000 + 12], [1, 12, 1, 5, 12], 48, 8, 128),
    # 6/1 heads: verify rows next to an 11-token chunk (66 rows)
    ("mqa_rows66_verify", [20000 + 6, 20000 + 11, 9000 + 6], [6, 11, 6], 6, 1, 128),
]

# fresh prompts: 1, 2 and 3 key tiles (ntk odd and even for both groups)
SHORT = [
    ("fresh12_ntk1", [12], [12], 48, 8),
    ("ctx70_ntk2", [70 + 12], [12], 48, 8),
    ("ctx150_ntk3", [150 + 12], [12], 48, 8),
    ("fresh100_g1", [100], [100], 8, 8),
]


def _header(ws, b):
    """(work items, split row tiles) left in the workspace, and the plan."""
    info = gfx906_fa.plan_info(b.num_seqs, b.num_tokens, b.Hq, b.Hkv, b.max_query_len, b.max_seq_len)
    off = info["pf_header_offset"]
    assert off >= 0, "the call has no prefill work list"
    hdr = ws[off:off + 8].view(torch.int32).cpu().tolist()
    return hdr[0], hdr[1], info


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_rows_class_matches_oracle(case):
    need_gpu()
    name, sls, qls, Hq, Hkv, rows = case
    announce(f"prefill rows {name}")
    b = W.build_batch(sls, qls, Hq, Hkv, seed=sum(map(ord, name)))
    ws = gfx906_fa.new_workspace(gfx906_fa.workspace_size(b.num_seqs, b.num_tokens, Hq, Hkv, b.max_query_len,
                                                          b.max_seq_len), DEV)
    out = W.attention(b, out_dtype=torch.float32, workspace=ws)
    torch.cuda.synchronize()
    items, nsplit, info = _header(ws, b)
    assert info["pf_rows"] == rows, info
    G = Hq // Hkv
    tiles = sum(-(-q * G // rows) for q in qls if q * G > info["dec_rows_max"])
    assert items >= tiles, (items, tiles)
    assert_close(to_np_f32(out), batch_oracle(b))


@pytest.mark.parametrize("case", SHORT, ids=[c[0] for c in SHORT])
def test_rows128_short_contexts(case):
    """Too few key tiles to split: one workgroup per row tile writes the output
    itself (no partial slots), with groups A and B padding their barriers."""
    need_gpu()
    name, sls, qls, Hq, Hkv = case
    announce(f"prefill rows128 {name}")
    b = W.build_batch(sls, qls, Hq, Hkv, seed=sum(map(ord, name)))
    ws = gfx906_fa.new_workspace(gfx906_fa.workspace_size(b.num_seqs, b.num_tokens, Hq, Hkv, b.max_query_len,
                                                          b.max_seq_len), DEV)
    out = W.attention(b, out_dtype=torch.float32, workspace=ws)
    torch.cuda.synchronize()
    items, nsplit, info = _header(ws, b)
    assert info["pf_rows"] == 128, info
    assert nsplit == 0, nsplit
    assert_close(to_np_f32(out), batch_oracle(b))


def test_rows128_split_and_whole():
    """The same 72-row chunk on a long context (split over the keys: partial
    slots of 128 rows, merged by the combine kernel) and on a short one
    (whole)."""
    need_gpu()
    announce("prefill rows128 split vs whole")
    for sl, want_split in ((60000 + 12, True), (400 + 12, False)):
        b = W.build_batch([sl], [12], 48, 8, seed=sl)
        ws = gfx906_fa.new_workspace(gfx906_fa.workspace_size(b.num_seqs, b.num_tokens, 48, 8, b.max_query_len,
                                                              b.max_seq_len), DEV)
        out = W.attention(b, out_dtype=torch.float32, workspace=ws)
        torch.cuda.synchronize()
        items, nsplit, info = _header(ws, b)
        assert info["pf_rows"] == 128
        assert (nsplit > 0) == want_split, (sl, nsplit)
        assert_close(to_np_f32(out), batch_oracle(b))


@pytest.mark.parametrize("dt,extra", [(torch.float16, 2.0 ** -11), (torch.bfloat16, 2.0 ** -8)])
def test_rows128_output_dtypes(dt, extra):
    need_gpu()
    announce(f"prefill rows128 out={dt}")
    b = W.build_batch([6000 + 12, 3000 + 20], [12, 20], 48, 8, seed=191)
    out = W.attention(b, out_dtype=dt)
    torch.cuda.synchronize()
    assert out.dtype == dt
    assert_close(to_np_f32(out), batch_oracle(b), extra=extra)


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_rows128_query_dtypes(dtype):
    need_gpu()
    announce(f"prefill rows128 query={dtype}")
    b = W.build_batch([5000 + 14], [14], 48, 8, dtype=dtype, seed=194)
    out = W.attention(b)
    torch.cuda.synchronize()
    assert out.dtype == b.query.dtype
    extra = {"bf16": 2.0 ** -8, "f32": 0.0}[dtype]
    assert_close(to_np_f32(out), batch_oracle(b), extra=extra)


def test_rows128_q_abs_offset():
    """A 12-token chunk at position 3000 of a 7000-token sequence: keys past
    each row's bound exist in the cache but stay masked."""
    need_gpu()
    announce("prefill rows128 q_abs_offset")
    b = W.build_batch([7000], [12], 48, 8, seed=195)
    kp, vp = b.planes()
    qa = np.array([3000], np.int32)
    out = gfx906_fa.paged_attention(b.query, kp, vp, b.block_table, b.seq_lens_t, b.qsl_t, b.max_query_len,
                                    b.max_seq_len, b.scale, out_dtype=torch.float32,
                                    q_abs_offset=torch.from_numpy(qa).to(DEV))
    torch.cuda.synchronize()
    assert_close(to_np_f32(out), batch_oracle(b, q_abs=qa))
