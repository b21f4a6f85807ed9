"""GPU: attention on the layouts a serving engine hands over.

- GQA ratios that do not divide 16 (G = 3, 5, 7): the packed row -> (token,
  q-head) mapping in the 16-row and 32-row decode classes and in prefill.
- Prefix caching: sequences whose block tables share pages (the same block
  ids), read by several sequences in one batch.
- Strided views: the query as a slice of a fused QKV tensor, the output as a
  slice of a wider buffer; results equal the contiguous call bit for bit.
Each case is checked against the oracle, as in tests/test_gpu_attention.py."""
import numpy as np
import pytest
import torch

import gfx906_fa
import gfx906_fa_workloads as W
from gpu_common import announce, assert_close, batch_oracle, need_gpu, to_np_f32

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _check(b, out_dtype=torch.float32):
    out = W.attention(b, out_dtype=out_dtype)
    torch.cuda.synchronize()
    assert_close(to_np_f32(out), batch_oracle(b))
    return out


@pytest.mark.parametrize("G", [3, 5, 7])
def test_gqa_ratios_not_dividing_16(G):
    """Per G: n_q = 1..3 put G..3G rows in the decode classes, 5 (15, 25, 35
    rows) straddles them, and a 100-token chunk goes to prefill."""
    need_gpu()
    announce(f"gqa G={G}")
    hkv = 2
    b = W.build_batch([40, 700, 1500, 33, 900, 260], [1, 2, 3, 5, 5, 100], G * hkv, hkv, seed=50 + G)
    _check(b)


def test_shared_prefix_pages():
    """Sequences 1 and 2 reuse sequence 0's first pages (as vLLM's prefix
    cache does); every sequence reads its pages through its own table."""
    need_gpu()
    announce("shared prefix pages")
    b = W.build_batch([1000, 1200, 800, 300], [1, 5, 64, 1], 12, 2, seed=60)
    bt = b.block_table_np.copy()
    shared = 800 // b.block_size  # pages of the first 800 tokens
    bt[1, :shared] = bt[0, :shared]
    bt[2, :shared] = bt[0, :shared]
    b.block_table_np = bt
    b.block_table = torch.from_numpy(bt).to(DEV)
    _check(b)


def test_strided_query_and_output_views():
    need_gpu()
    announce("strided query / output")
    b = W.build_batch([500, 37, 2000, 64], [1, 37, 5, 64], 16, 4, seed=70)
    kp, vp = b.planes()
    T, Hq, D, Hkv = b.num_tokens, b.Hq, b.D, b.Hkv
    qkv = torch.zeros((T, Hq + 2 * Hkv, D), dtype=b.query.dtype, device=DEV)
    qkv[:, :Hq] = b.query
    q_view = qkv[:, :Hq]
    assert not q_view.is_contiguous()
    wide = torch.full((T, Hq + 3, D), -7.0, dtype=torch.float16, device=DEV)
    o_view = wide[:, 1:Hq + 1]
    args = (kp, vp, b.block_table, b.seq_lens_t, b.qsl_t, b.max_query_len, b.max_seq_len, b.scale)
    ref = gfx906_fa.paged_attention(b.query, *args, out_dtype=torch.float16)
    gfx906_fa.paged_attention(q_view, *args, out=o_view)
    torch.cuda.synchronize()
    assert torch.equal(o_view, ref)
    assert bool((wide[:, 0] == -7.0).all()) and bool((wide[:, Hq + 1:] == -7.0).all())
    assert_close(to_np_f32(ref), batch_oracle(b), extra=2.0 ** -11)
