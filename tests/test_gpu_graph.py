"""GPU: a decode step (quantize-write of the new tokens + paged attention)
captured once in a HIP graph and replayed with new sequence lengths, block
tables and token values written in place.  Every replay is checked bit for
bit against the same step run eagerly (with the program's own eager work and
synchronisations between replays), and one replay against the oracle.  The
attention path allocates nothing inside the C ABI, records no memset, and
sizes its grids from host-fixed shapes only (CU count, num_seqs, heads,
max_query_len), so the graph stays valid while the device-side metadata
changes.  A prefill call that writes the tile images is captured and
replayed the same way."""
import math

import numpy as np
import pytest
import torch

import gfx906_fa
from gpu_common import announce, assert_close, need_gpu
from oracle import q8_oracle as O

DEV = "cuda"
pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("fused", [False, True])
@pytest.mark.parametrize("heads,q_len,max_blocks", [((48, 8), 1, 48), ((6, 1), 5, 48), ((6, 1), 6, 48),
                                                   ((6, 1), 6, 640)])
def test_decode_step_graph_replay(heads, q_len, max_blocks, fused):
    """fused: the cache write folded into the attention call.  6 tokens at
    6/1 (36 rows) take two 32-row chunks at 768-token contexts and 48-row
    tiles at 10240."""
    need_gpu()
    Hq, Hkv = heads
    announce(f"graph replay heads={heads} q_len={q_len} max_blocks={max_blocks} fused={fused}")
    B, bs = 8, 16
    NB = B * max_blocks
    T = B * q_len
    scale = 1.0 / math.sqrt(128)
    rng = np.random.default_rng(5)
    cache = gfx906_fa.new_kv_cache(NB, bs, Hkv, device=DEV)
    kp, vp = cache[:, 0], cache[:, 1]
    # fill every page once (eager) so any block table reads written data
    allk = torch.from_numpy(rng.standard_normal((NB * bs, Hkv, 128)).astype(np.float16)).to(DEV)
    allv = torch.from_numpy(rng.standard_normal((NB * bs, Hkv, 128)).astype(np.float16)).to(DEV)
    gfx906_fa.reshape_and_cache_q8_kv(allk, allv, torch.arange(NB * bs, dtype=torch.int64, device=DEV), kp, vp)
    # static graph inputs / outputs
    q = torch.empty((T, Hq, 128), dtype=torch.float16, device=DEV)
    k_new = torch.empty((T, Hkv, 128), dtype=torch.float16, device=DEV)
    v_new = torch.empty_like(k_new)
    slots = torch.empty(T, dtype=torch.int64, device=DEV)
    bt = torch.empty((B, max_blocks), dtype=torch.int32, device=DEV)
    sl = torch.empty(B, dtype=torch.int32, device=DEV)
    qsl = torch.arange(0, (B + 1) * q_len, q_len, dtype=torch.int32, device=DEV)
    out = torch.empty((T, Hq, 128), dtype=torch.float16, device=DEV)
    ws = gfx906_fa.new_workspace(gfx906_fa.workspace_size(B, T, Hq, Hkv, q_len, max_blocks * bs), DEV)

    def load_inputs(seed):
        r = np.random.default_rng(seed)
        lens = r.integers(q_len, max_blocks * bs + 1, B).astype(np.int32)
        table = r.permutation(NB)[: B * max_blocks].astype(np.int32).reshape(B, max_blocks)
        pos = (lens[:, None] - q_len + np.arange(q_len)[None, :]).reshape(-1)
        rows = np.repeat(np.arange(B), q_len)
        sm = table[rows, pos // bs].astype(np.int64) * bs + pos % bs
        sl.copy_(torch.from_numpy(lens))
        bt.copy_(torch.from_numpy(table))
        slots.copy_(torch.from_numpy(sm))
        q.copy_(torch.from_numpy(r.standard_normal((T, Hq, 128)).astype(np.float16)))
        k_new.copy_(torch.from_numpy(r.standard_normal((T, Hkv, 128)).astype(np.float16)))
        v_new.copy_(torch.from_numpy(r.standard_normal((T, Hkv, 128)).astype(np.float16)))
        return lens, table

    def step():
        if fused:
            gfx906_fa.paged_attention(q, kp, vp, bt, sl, qsl, q_len, max_blocks * bs, scale, out=out,
                                      workspace=ws, new_key=k_new, new_value=v_new, slot_mapping=slots)
            return
        gfx906_fa.reshape_and_cache_q8_kv(k_new, v_new, slots, kp, vp)
        gfx906_fa.paged_attention(q, kp, vp, bt, sl, qsl, q_len, max_blocks * bs, scale, out=out, workspace=ws)

    load_inputs(100)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()  # warm-up outside capture
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step()
    for it in range(4):
        lens, table = load_inputs(200 + it)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        got = out.clone()
        step()  # eager, same inputs (the cache write is idempotent)
        torch.cuda.synchronize()
        assert torch.equal(got, out), f"replay {it} differs from the eager step"
        if it == 3:
            kh, vh = O.planar_dequant(cache.cpu().numpy())
            ref = O.paged_attention_ref(q.float().cpu().numpy(), kh, vh, table, lens,
                                        qsl.cpu().numpy(), scale)
            assert_close(got.float().cpu().numpy(), ref)


def test_prefill_with_tile_images_graph_replay():
    """A prefill call whose plan writes the tile images (a 3000-token prompt
    at 48/8: plan kernel, image pre-pass, prefill and split-merge launches)
    captured once and replayed three times with new query values written in
    place and eager calls in between; every replay equals the eager call bit
    for bit, and the work-list header says the images were written."""
    need_gpu()
    import gfx906_fa_workloads as W
    announce("graph replay prefill with tile images, 3000 tokens 48/8")
    b = W.build_batch([3000], [3000], 48, 8, dtype="bf16", seed=81)
    kp, vp = b.planes()
    info = gfx906_fa.plan_info(b.num_seqs, b.num_tokens, b.Hq, b.Hkv, b.max_query_len, b.max_seq_len)
    ws = gfx906_fa.new_workspace(info["bytes"], b.device)
    out = torch.empty((b.num_tokens, b.Hq, 128), dtype=torch.float32, device=DEV)

    def call():
        gfx906_fa.paged_attention(b.query, kp, vp, b.block_table, b.seq_lens_t, b.qsl_t, b.max_query_len,
                                  b.max_seq_len, b.scale, out=out, workspace=ws)

    call()
    torch.cuda.synchronize()
    hdr = ws[info["pf_header_offset"]:info["pf_header_offset"] + 16].view(torch.int32).cpu().tolist()
    assert hdr[2] == 1 and hdr[3] > 0, hdr
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        call()  # warm-up on the capture stream
        torch.cuda.synchronize()
        with torch.cuda.graph(g, stream=s):
            call()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    gen = torch.Generator(device="cpu").manual_seed(82)
    for it in range(3):
        newq = torch.randn(b.query.shape, generator=gen, dtype=torch.float32).to(dtype=b.query.dtype, device=DEV)
        b.query.copy_(newq)
        call()  # eager reference, then the replay over the same inputs
        torch.cuda.synchronize()
        ref = out.clone()
        out.fill_(7.0)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"replay {it} differs from the eager call"
