"""GPU: prefill tiles dequantized once into the workspace (tile images copied
into LDS by the prefill workgroups) against the same calls with a workspace
that has no room for them (every workgroup dequantizes its tiles): the
outputs are equal bit for bit, the work-list header says which path ran, and
one shape is also checked against the float64 oracle.  The plan writes the
images only where the row tiles read each key tile at least 32 times on
average (a prompt of 64 or more row tiles); every image shape here does.
Shapes: a long prompt, a prompt with one query head per kv head whose row
tiles are split over the keys (pieces start past key tile 0), block size 64,
a mixed batch with decode sequences, explicit query positions without the
causal mask; and a short chunk on a long prefix, read about twice per tile,
which gets no image room (no sequence has 32 row tiles), and a 40-row-tile
prompt, which gets the room but whose row tiles read each key tile about
20 times on average, so the plan keeps the in-kernel dequantization
(reference: tests/test_inline_causal.py, tests/test_fa_mixed_batch.py)."""
import numpy as np
import pytest
import torch

import gfx906_fa
import gfx906_fa_workloads as W
from gpu_common import announce, assert_close, batch_oracle, need_gpu, to_np_f32

pytestmark = pytest.mark.gpu

CASES = [
    # name, seq_lens, q_lens, Hq, Hkv, block_size, dtype, images written
    ("prompt 3000", [3000], [3000], 48, 8, 16, "bf16", True),
    ("split prompt G=1", [20000], [20000], 2, 2, 16, "f16", True),
    ("bs64 G=1", [20000, 3000], [20000, 3000], 4, 4, 64, "f16", True),
    ("mixed with decodes", [4000, 70, 5000, 333, 1200], [400, 1, 5000, 5, 1], 32, 4, 32, "bf16", True),
    ("chunk on a long prefix", [20000 + 60], [60], 48, 8, 16, "f16", False),
    ("prompt below the reuse bar", [10240], [10240], 1, 1, 16, "f16", False),
]


def _header(ws, off):
    return ws[off:off + 16].view(torch.int32).cpu().tolist()


def _run(b, nbytes, q_abs=None, causal=True):
    kp, vp = b.planes()
    ws = gfx906_fa.new_workspace(nbytes, b.device)
    out = gfx906_fa.paged_attention(b.query, kp, vp, b.block_table, b.seq_lens_t, b.qsl_t, b.max_query_len,
                                    b.max_seq_len, b.scale, workspace=ws, q_abs_offset=q_abs, causal=causal,
                                    out_dtype=torch.float32)
    torch.cuda.synchronize()
    return out, ws


def _both(b, q_abs=None, causal=True, images=True):
    info = gfx906_fa.plan_info(b.num_seqs, b.num_tokens, b.Hq, b.Hkv, b.max_query_len, b.max_seq_len)
    assert info["prefill"] == 1 and info["pf_header_offset"] >= 0
    assert (info["img_bytes"] > 0) == (b.max_query_len * b.Hq // b.Hkv > 31 * 256), info
    out_i, ws_i = _run(b, info["bytes"], q_abs, causal)
    out_d, ws_d = _run(b, info["img_offset"], q_abs, causal)
    hi, hd = _header(ws_i, info["pf_header_offset"]), _header(ws_d, info["pf_header_offset"])
    if images:
        assert hi[2] == 1 and hi[3] > 0, hi   # images written and copied
    else:
        assert hi[2] == 0 and hi[3] == 0, hi  # too little reuse: no images
    assert hd[2] == 0, hd                     # no room: dequantized in the workgroups
    assert hi[0] == hd[0] and hi[1] == hd[1]  # the same work list
    assert torch.equal(out_i, out_d)
    return out_i


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_images_equal_in_kernel_dequant(case):
    need_gpu()
    name, sl, ql, hq, hkv, bs, dt, images = case
    announce(f"prefill images {name}")
    b = W.build_batch(sl, ql, hq, hkv, block_size=bs, dtype=dt, seed=77 + len(name))
    _both(b, images=images)


def test_images_explicit_positions_not_causal():
    need_gpu()
    announce("prefill images q_abs, causal=False")
    b = W.build_batch([3000, 2000], [1500, 2000], 24, 4, dtype="f16", seed=91)
    q_abs = torch.tensor([700, 0], dtype=torch.int32, device=b.device)
    _both(b, q_abs=q_abs, causal=False)


def test_images_match_oracle():
    need_gpu()
    announce("prefill images vs oracle")
    b = W.build_batch([1100, 90], [1100, 1], 16, 1, block_size=32, dtype="bf16", seed=92)
    out = _both(b)
    assert_close(to_np_f32(out), batch_oracle(b))
