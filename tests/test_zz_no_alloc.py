"""GPU: the allocation-free attention entry point.

gfx906_fa_amd_paged_attention_noalloc (called through the C ABI) against
gfx906_fa_amd_paged_attention with a caller workspace, on two calls in a row
whose second is smaller (the library's scratch keeps the first call's
contents): decode and speculative-verify batches bit-identical (same plan),
prefill batches whose split partials would not fit the scratch within the
attention tolerance (unsplit row tiles: another summation order)."""
import ctypes

import numpy as np
import pytest
import torch

import gfx906_fa
import gfx906_fa_workloads as W
from gpu_common import announce, assert_close, batch_oracle, need_gpu, stream_ptr, to_np_f32

pytestmark = pytest.mark.gpu
DEV = "cuda"
_DT = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}


def _noalloc_fn():
    L = gfx906_fa.lib()
    f = L.gfx906_fa_amd_paged_attention_noalloc
    P, I, I64, F = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_float
    f.argtypes = [P, I, I64, I64, P, P, I64, I64, P, I64, P, P, P, I, I, I, I, I, I, I, I, I, F, P, I, I64, I64, P]
    f.restype = I
    return f


def _noalloc(b, out):
    kp, vp = b.planes()
    q = b.query
    err = _noalloc_fn()(q.data_ptr(), _DT[q.dtype], q.stride(0), q.stride(1), kp.data_ptr(), vp.data_ptr(),
                        kp.stride(0), kp.stride(1), b.block_table.data_ptr(), b.block_table.stride(0),
                        b.seq_lens_t.data_ptr(), b.qsl_t.data_ptr(), None, 1, b.num_seqs, b.num_tokens, b.Hq,
                        b.Hkv, 128, b.block_size, b.max_query_len, b.max_seq_len, b.scale, out.data_ptr(),
                        _DT[out.dtype], out.stride(0), out.stride(1), stream_ptr())
    assert err == 0, f"noalloc entry returned {err}"


def _scratch_header(b):
    """The prefill work-list header the last noalloc call left in the
    library's scratch: (items, split row tiles, images written, image tiles)."""
    off = gfx906_fa.plan_info(b.num_seqs, b.num_tokens, b.Hq, b.Hkv, b.max_query_len,
                              b.max_seq_len)["pf_header_offset"]
    assert off >= 0, "the call has no prefill work list"
    hdr = torch.zeros(4, dtype=torch.int32, device=DEV)
    err = gfx906_fa.lib().gfx906_fa_amd_noalloc_scratch_copy(hdr.data_ptr(), off, 16, stream_ptr())
    assert err == 0
    torch.cuda.synchronize()
    return hdr.cpu().tolist()


def _with_workspace(b, dt):
    out = torch.empty((b.num_tokens, b.Hq, 128), dtype=dt, device=DEV)
    W.attention(b, out=out)
    return out


@pytest.mark.parametrize("dt", [torch.float32, torch.float16])
def test_noalloc_decode_bitidentical(dt):
    """cfg2-like decode (48/8) then a smaller 6/1 verify batch: the scratch
    reused across calls, outputs equal the workspace entry's bit for bit."""
    need_gpu()
    rng = np.random.default_rng(70)
    big = W.build_batch(rng.integers(2048, 6000, 24).tolist(), [1] * 24, 48, 8, seed=71)
    small = W.build_batch([3000, 17, 900], [5, 5, 5], 6, 1, seed=72)
    for name, b in (("decode 24 x 48/8", big), ("verify 3 x 5 tokens 6/1", small)):
        announce(f"noalloc {name} {dt}")
        ref = _with_workspace(b, dt)
        out = torch.full_like(ref, 3.0)
        _noalloc(b, out)
        torch.cuda.synchronize()
        assert torch.equal(out, ref), name


def test_noalloc_48_row_tiles_bitidentical():
    """6-token verify at 6/1 (36 rows: the 48-row class), then a smaller
    batch mixing 5-, 6- and 1-token sequences (16-, 32- and 48-row classes in
    one call): bit-identical to the workspace entry."""
    need_gpu()
    first = W.build_batch([40000, 40, 2500, 700], [6] * 4, 6, 1, seed=76)
    second = W.build_batch([30000, 800, 1200], [5, 6, 1], 6, 1, seed=77)
    for name, b in (("verify 4 x 6 tokens 6/1", first), ("mixed 5/6/1 tokens 6/1", second)):
        announce(f"noalloc {name}")
        ref = _with_workspace(b, torch.float32)
        out = torch.full_like(ref, 3.0)
        _noalloc(b, out)
        torch.cuda.synchronize()
        assert torch.equal(out, ref), name


def test_noalloc_prefill_and_mixed():
    """A prefix-cached chunk whose row tiles the workspace entry splits over
    the keys (its partials would not fit the scratch: unsplit here), then a
    smaller mixed decode + prefill batch; both against the workspace entry
    and the oracle at the attention tolerance."""
    need_gpu()
    big = W.build_batch([8192 + 50], [50], 48, 8, seed=73)
    small = W.build_batch([700, 33, 1500, 260], [1, 33, 200, 5], 16, 2, seed=74)
    for name, b in (("chunk 50 on 8192, 48/8", big), ("mixed 4 seqs 16/2", small)):
        announce(f"noalloc {name}")
        ref = _with_workspace(b, torch.float32)
        out = torch.full_like(ref, 3.0)
        _noalloc(b, out)
        torch.cuda.synchronize()
        if b is big:
            assert _scratch_header(b)[1] == 0  # the row tiles ran unsplit
        assert_close(to_np_f32(out), to_np_f32(ref))
        assert_close(to_np_f32(out), batch_oracle(b))


def test_noalloc_prompt_with_tile_images():
    """A 3000-token prompt at 48/8: its row tiles read each key tile about 37
    times, so the plan writes the 64-key tile images (13.5 MB, room the
    scratch has past this unsplit plan); the output equals the workspace
    entry's (which takes the same path) bit for bit."""
    need_gpu()
    announce("noalloc prompt 3000 48/8 with tile images")
    b = W.build_batch([3000], [3000], 48, 8, dtype="bf16", seed=75)
    ref = _with_workspace(b, torch.float32)
    out = torch.full_like(ref, 3.0)
    _noalloc(b, out)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
    hdr = _scratch_header(b)
    assert hdr[2] == 1 and hdr[3] > 0, hdr  # the images were written in the scratch


def test_noalloc_rows128_bitidentical():
    """Chunks of 12 tokens at 48/8 (72 rows per kv-head: the 128-row
    key-interleaved prefill tiles), on a long prefix and then a shorter one:
    the noalloc entry takes the workspace entry's plan where its split
    partials fit the scratch, so the output is the same bits."""
    need_gpu()
    first = W.build_batch([20000 + 12, 900 + 12], [12, 12], 48, 8, seed=78)
    second = W.build_batch([3000 + 12], [12], 48, 8, seed=79)
    for name, b in (("2 chunks of 12 on 20K / 900, 48/8", first), ("1 chunk of 12 on 3K", second)):
        announce(f"noalloc rows128 {name}")
        info = gfx906_fa.plan_info(b.num_seqs, b.num_tokens, 48, 8, b.max_query_len, b.max_seq_len)
        assert info["pf_rows"] == 128 and info["img_offset"] <= 64 << 20, info
        ref = _with_workspace(b, torch.float32)
        out = torch.full_like(ref, 3.0)
        _noalloc(b, out)
        torch.cuda.synchronize()
        assert torch.equal(out, ref), name
        if b is first:
            assert _scratch_header(b)[1] > 0  # split over the keys, as with a workspace
