"""GPU: direct-paged attention vs the dequantize-then-float64 oracle.

Tolerance (north star): max-abs 2e-3 and relative Frobenius error 1e-2 for
fp32 outputs; fp16 / bf16 outputs additionally allow their own rounding
(2^-11 / 2^-8 of |ref|).  Cases follow the reference's tests:
decode batches (tests/test_decode_batch.py, test_direct_paged_bitexact.py),
inline-causal chunked prefill (tests/test_inline_causal.py), mixed batches
and the TP-8 shard (tests/test_fa_mixed_batch.py), the backend end to end
(tests/test_backend.py), plus split-K, GQA, block sizes, dtypes, empty
sequences, and full-size configurations checked on sampled rows and by
block-table permutation invariance."""
import math
import os

import numpy as np
import pytest
import torch

import gfx906_fa
import gfx906_fa_workloads as W
from gpu_common import announce, assert_close, batch_oracle, need_gpu, to_np_f32
from oracle import q8_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"
ROUND = {torch.float32: 0.0, torch.float16: 2.0 ** -11, torch.bfloat16: 2.0 ** -8}


def _run_and_check(b, out_dtype=torch.float32, rows=None):
    announce(f"attention B={b.num_seqs} T={b.num_tokens} Hq={b.Hq} Hkv={b.Hkv} bs={b.block_size} "
             f"max_q={b.max_query_len} max_k={b.max_seq_len} {b.dtype}->{out_dtype}")
    out = W.attention(b, out_dtype=out_dtype)
    torch.cuda.synchronize()
    ref = batch_oracle(b, rows=rows)
    got = to_np_f32(out)
    if rows is not None:
        got, ref = got[rows], ref[rows]
    assert_close(got, ref, extra=ROUND[out_dtype])
    return out


def test_golden_cfg1():
    """The committed cfg1 fixture: cache bytes bit-exact, output in tolerance."""
    need_gpu()
    announce("golden cfg1")
    g = np.load(os.path.join(os.path.dirname(__file__), "golden", "q8_cfg1.npz"))
    nb, bs = int(g["num_blocks"]), int(g["block_size"])
    cache = gfx906_fa.new_kv_cache(nb, bs, 1, device=DEV)
    key = torch.from_numpy(g["key"]).to(DEV)
    val = torch.from_numpy(g["value"]).to(DEV)
    gfx906_fa.reshape_and_cache_q8_kv(key, val, torch.from_numpy(g["slot_mapping"]).to(DEV),
                                      cache[:, 0], cache[:, 1])
    assert np.array_equal(cache.cpu().numpy(), g["cache"])
    q = torch.from_numpy(g["query"]).to(DEV)
    out = gfx906_fa.paged_attention(q, cache[:, 0], cache[:, 1], torch.from_numpy(g["block_table"]).to(DEV),
                                    torch.from_numpy(g["seq_lens"]).to(DEV),
                                    torch.from_numpy(g["query_start_loc"]).to(DEV), 1, 1024,
                                    1.0 / math.sqrt(128), out_dtype=torch.float32)
    assert_close(to_np_f32(out), g["out"])


@pytest.mark.parametrize("heads", [(8, 1), (48, 8), (32, 4), (16, 16)])
@pytest.mark.parametrize("dt", ["f16", "bf16"])
def test_decode_batch(heads, dt):
    need_gpu()
    hq, hkv = heads
    b = W.build_batch([1, 15, 16, 17, 300, 1000, 2049], [1] * 7, hq, hkv, dtype=dt, seed=1)
    _run_and_check(b)


def test_decode_split_k_long():
    """Long contexts force several splits and the combine kernel."""
    need_gpu()
    b = W.build_batch([20000, 777, 12345], [1] * 3, 8, 1, seed=2)
    _run_and_check(b)


@pytest.mark.parametrize("bs", [32, 64])
def test_decode_block_sizes(bs):
    need_gpu()
    b = W.build_batch([5, 100, 1500], [1] * 3, 12, 2, block_size=bs, seed=3)
    _run_and_check(b)


@pytest.mark.parametrize("bs", [128, 256])
def test_mixed_batch_large_blocks(bs):
    """Pages of 8 and 16 sub-pages, through both the decode and the prefill
    kernel (vLLM's block size is any multiple of 16)."""
    need_gpu()
    b = W.build_batch([5, 300, 1500, 700, 33], [1, 1, 1, 300, 33], 12, 2, block_size=bs, seed=31)
    _run_and_check(b)


@pytest.mark.parametrize("nq", [1, 2, 3])
def test_gqa_16(nq):
    """G = 16 (64/4 heads): one query token fills the 16-row decode tile,
    two fill the 32-row tile, three (48 rows) go to the prefill kernel."""
    need_gpu()
    b = W.build_batch([40, 900, 3001], [nq] * 3, 64, 4, seed=32 + nq)
    _run_and_check(b)


def test_decode_many_sequences():
    """300 sequences: the device-side plan scans run over several 64-wide
    chunks of sequences, and contexts of 1..600 tokens leave many segments
    whole inside one workgroup and others split."""
    need_gpu()
    rng = np.random.default_rng(33)
    b = W.build_batch(rng.integers(1, 601, 300), [1] * 300, 8, 1, seed=33)
    _run_and_check(b)


def test_prefill_mha_several_row_tiles():
    """G = 1 (16/16 heads): a 600-token prefill spans three 256-row tiles;
    lengths off the 16-token grid."""
    need_gpu()
    b = W.build_batch([600, 257], [600, 250], 16, 16, seed=34)
    _run_and_check(b)


def test_inline_causal_chunked_prefill():
    """tests/test_inline_causal.py: 8/2 heads, seq 512/384, chunks 256/128."""
    need_gpu()
    b = W.build_batch([512, 384], [256, 128], 8, 2, seed=4)
    _run_and_check(b)


@pytest.mark.parametrize("dt", ["f16", "bf16"])
def test_full_prefill(dt):
    need_gpu()
    b = W.build_batch([300, 77], [300, 77], 12, 2, dtype=dt, seed=5)
    _run_and_check(b)


def test_mixed_batch():
    need_gpu()
    sl = [64, 700, 1500, 33, 4000, 9]
    ql = [64, 200, 1, 1, 1, 9]
    b = W.build_batch(sl, ql, 48, 8, seed=6)
    _run_and_check(b)


@pytest.mark.parametrize("heads", [(6, 1), (48, 8)])
def test_spec_verify(heads):
    """5 verify tokens causal among themselves (G*5 = 30 rows)."""
    need_gpu()
    b = W.build_batch([3000, 5, 1200], [5, 5, 5], heads[0], heads[1], seed=7)
    _run_and_check(b)


def test_verify_more_rows_than_decode_tile():
    """n_q*G = 48 > 32 rows: the three-row-group launch takes them in one
    48-row tile per wave (long enough contexts: at least 8 sub-pages per
    workgroup)."""
    need_gpu()
    b = W.build_batch([40000, 40], [8, 8], 6, 1, seed=8)
    _run_and_check(b)


@pytest.mark.parametrize("case", [
    ("6 tokens 6/1", [3000, 6, 1200, 17, 20000], [6] * 5, 6, 1, 16),      # 36 rows
    ("7 tokens 6/1", [5000, 300, 64], [7] * 3, 6, 1, 16),                 # 42 rows
    ("8 tokens 8/1", [2500, 9, 4100], [8] * 3, 8, 1, 16),                 # 64 rows
    ("64/1 heads", [700, 33, 3000], [1] * 3, 64, 1, 16),                  # G = 64: 64 rows
    ("mixed 5/6 tokens", [30000, 800, 1200, 40], [5, 6, 1, 6], 6, 1, 16),  # 16-, 32- and 48-row classes
    ("mixed 5/6 tokens short", [3000, 800, 1200, 40], [5, 6, 1, 6], 6, 1, 16),  # 16-row and chunked classes
    ("6 tokens 48/8 bs64", [2000, 6000, 333], [6] * 3, 48, 8, 64),
    ("mixed 1/5/8 tokens 8/1", [3000, 900, 2500, 70], [1, 5, 8, 5], 8, 1, 16),  # 16-row and chunked classes
    ("5 tokens 64/8", [4000, 12, 900], [5] * 3, 64, 8, 16),              # 40 rows per kv-head
    # 96 segments: the verify class of a mixed batch merges one segment per workgroup
    ("verify + chunk 48/8", [20000] * 8 + [3000, 50, 9000, 5000], [6] * 8 + [1, 1, 1, 300], 48, 8, 16),
])
def test_verify_rows_33_to_64(case):
    """Speculative verify with num_speculative_tokens = 5 (6 query tokens, the
    reference's n-gram setting, scripts/start_vllm_fa_ngram.sh:35-39) packs
    36 rows per kv-head at 6 q-heads: the decode kernel takes up to 48 rows
    in one tile per wave (three 16-row groups) and up to 64 rows in two
    32-row chunks, instead of sending them to the prefill kernel."""
    need_gpu()
    name, sl, ql, hq, hkv, bs = case
    b = W.build_batch(sl, ql, hq, hkv, block_size=bs, seed=80 + len(name))
    _run_and_check(b)


@pytest.mark.parametrize("odt", [torch.float16, torch.bfloat16])
def test_output_dtypes(odt):
    need_gpu()
    b = W.build_batch([100, 2000], [1, 50], 16, 2, seed=9)
    _run_and_check(b, out_dtype=odt)


def test_fp32_query():
    need_gpu()
    b = W.build_batch([260, 31], [1, 31], 8, 2, dtype="f32", seed=10)
    _run_and_check(b)


def test_empty_sequences():
    """seq_len 0 -> zeros; a sequence with no query tokens writes nothing."""
    need_gpu()
    announce("empty sequences")
    b = W.build_batch([50, 0, 30, 20], [1, 1, 0, 2], 8, 2, seed=11)
    sentinel = torch.full((b.num_tokens, 8, 128), 7.0, device=DEV)
    out = W.attention(b, out=sentinel)
    torch.cuda.synchronize()
    ref = batch_oracle(b)
    o = to_np_f32(out)
    assert not o[1].any()           # token of the seq_len 0 sequence
    assert_close(o, ref)


def test_zero_token_batch():
    """Every sequence with an empty query (num_tokens 0, whatever strides the
    empty query tensor has): an empty output and no launch."""
    need_gpu()
    announce("zero-token batch")
    b = W.build_batch([1467, 30], [0, 0], 12, 2, seed=12)
    assert b.num_tokens == 0
    out = W.attention(b, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert tuple(out.shape) == (0, 12, 128)
    q = torch.empty((0, 12, 128), dtype=torch.float16, device=DEV).as_strided((0, 12, 128), (0, 0, 0))
    kp, vp = b.planes()
    out = gfx906_fa.paged_attention(q, kp, vp, b.block_table, b.seq_lens_t, b.qsl_t, 0, b.max_seq_len, b.scale)
    assert out.numel() == 0


def test_forward_paged_direct_padded():
    """Reference-signature padded entry: non-causal (kv_max cutoff) and
    inline-causal via q_abs_offset (extension/gfx906_fa.cpp:516-658)."""
    need_gpu()
    announce("forward_paged_direct")
    b = W.build_batch([40, 200, 77], [1, 1, 1], 8, 2, seed=12)
    B, Sq = 3, 4
    q = torch.randn((B, 8, Sq, 128), device=DEV, dtype=torch.float32)
    kp, vp = b.planes()
    out = gfx906_fa.forward_paged_direct(q, kp, vp, b.block_table, b.seq_lens_t, b.scale)
    qo = torch.tensor([30, 100, 73], dtype=torch.int32, device=DEV)
    outc = gfx906_fa.forward_paged_direct(q, kp, vp, b.block_table, b.seq_lens_t, b.scale, q_abs_offset=qo)
    torch.cuda.synchronize()
    cache = b.kv_cache.cpu().numpy()
    kh, vh = O.planar_dequant(cache)
    qn = q.cpu().numpy()
    for s in range(B):
        for j in range(Sq):
            for causal, o in ((False, out), (True, outc)):
                lim = (int(qo[s]) + j + 1) if causal else int(b.seq_lens[s])
                lim = min(lim, int(b.seq_lens[s]))
                ref = O.paged_attention_ref(qn[s, :, j][None], kh, vh, b.block_table_np[s:s + 1],
                                            np.array([lim], np.int32), np.array([0, 1], np.int32), b.scale)
                assert_close(o[s, :, j].cpu().numpy(), ref[0])


def test_backend_impl_end_to_end():
    """tests/test_backend.py:60-162 with the vllm stub: do_kv_cache_update then
    forward on a vLLM-shaped [NB, 2, bs, Hkv, D] fp16 cache."""
    need_gpu()
    announce("backend impl end to end")
    from gfx906_fa_backend import Gfx906FAImpl, Gfx906FAMetadata
    Hq, Hkv, D, bs, NB = 8, 4, 128, 16, 8
    Sk = 64
    torch.manual_seed(0)
    kv = torch.zeros((NB, 2, bs, Hkv, D), dtype=torch.float16, device=DEV)
    impl = Gfx906FAImpl(Hq, D, 1 / math.sqrt(D), Hkv, None, None, "auto")
    bt = torch.tensor([[3, 0, 6, 1]], dtype=torch.int32, device=DEV)
    pos = torch.arange(Sk, device=DEV)
    slots = (bt[0, pos // bs].long() * bs + pos % bs)
    keys = torch.randn((Sk, Hkv, D), dtype=torch.float16, device=DEV)
    vals = torch.randn((Sk, Hkv, D), dtype=torch.float16, device=DEV)
    impl.do_kv_cache_update(None, keys[:-1], vals[:-1], kv, slots[:-1])   # prefix
    impl.do_kv_cache_update(None, keys[-1:], vals[-1:], kv, slots[-1:])   # the decode token
    q = torch.randn((1, Hq, D), dtype=torch.float16, device=DEV)
    md = Gfx906FAMetadata(num_actual_tokens=1, max_query_len=1, max_seq_len=Sk,
                          query_start_loc=torch.tensor([0, 1], dtype=torch.int32, device=DEV),
                          seq_lens=torch.tensor([Sk], dtype=torch.int32, device=DEV),
                          block_table=bt, slot_mapping=slots[-1:])
    output = torch.empty((1, Hq * D), dtype=torch.float16, device=DEV)
    res = impl.forward(None, q, keys[-1:], vals[-1:], kv, md, output=output)
    torch.cuda.synchronize()
    assert res is output
    kq = O.dequantize_q8_0_rows(O.quantize_q8_0_rows(keys.cpu().numpy()), 128)
    vq = O.dequantize_q8_0_rows(O.quantize_q8_0_rows(vals.cpu().numpy()), 128)
    qn = q.float().cpu().numpy()
    ref = np.zeros((Hq, D))
    for h in range(Hq):
        sc = kq[:, h // 2] @ qn[0, h] / math.sqrt(D)
        p = np.exp(sc - sc.max())
        ref[h] = p @ vq[:, h // 2] / p.sum()
    assert_close(output.float().cpu().numpy().reshape(Hq, D), ref, extra=2.0 ** -11)


@pytest.mark.parametrize("bs", [16, 32])
def test_backend_q8_0_pages_match_fp16_pages(bs):
    """The "q8_0" cache dtype (pages of exactly the Q8_0 planes) against the
    default fp16-sized pages: the same writes give the same plane bytes, and
    a mixed prefill + decode forward gives bit-identical outputs, in
    tolerance of the oracle."""
    need_gpu()
    announce(f"backend q8_0 pages vs fp16 pages bs={bs}")
    from gfx906_fa_backend import Gfx906FABackend, Gfx906FAImpl, Gfx906FAMetadata
    from gfx906_fa_paged import q8_planes
    Hq, Hkv, D, NB = 16, 4, 128, 40
    rng = np.random.default_rng(21)
    torch.manual_seed(21)
    sl = [300, 41, 170]
    ql = [300, 1, 5]
    nblk = [(n + bs - 1) // bs for n in sl]
    perm = rng.permutation(NB)[:sum(nblk)]
    bt = np.full((3, max(nblk)), -1, np.int32)
    o = 0
    for s, n in enumerate(nblk):
        bt[s, :n] = perm[o:o + n]
        o += n
    btt = torch.from_numpy(bt).to(DEV)
    caches = {}
    for cd in ("auto", "q8_0"):
        page = Gfx906FABackend.get_kv_cache_page_size_bytes(bs, Hkv, D, cd, torch.float16)
        raw = torch.zeros(page * NB, dtype=torch.int8, device=DEV)
        caches[cd] = raw.view(torch.uint8 if cd == "q8_0" else torch.float16).view(
            Gfx906FABackend.get_kv_cache_shape(NB, bs, Hkv, D, cd))
    keys = [torch.randn((n, Hkv, D), dtype=torch.float16, device=DEV) for n in sl]
    vals = [torch.randn((n, Hkv, D), dtype=torch.float16, device=DEV) for n in sl]
    slots = []
    for s, n in enumerate(sl):
        pos = torch.arange(n, device=DEV)
        slots.append(btt[s, pos // bs].long() * bs + pos % bs)
    q = torch.randn((sum(ql), Hq, D), dtype=torch.float16, device=DEV)
    qsl = torch.tensor(np.concatenate([[0], np.cumsum(ql)]), dtype=torch.int32, device=DEV)
    outs = {}
    for cd, kv in caches.items():
        impl = Gfx906FAImpl(Hq, D, 1 / math.sqrt(D), Hkv, None, None, cd)
        for s, n in enumerate(sl):       # context first, then the step's new tokens
            k = ql[s]
            impl.do_kv_cache_update(None, keys[s][:n - k], vals[s][:n - k], kv, slots[s][:n - k])
        nk = torch.cat([keys[s][n - ql[s]:] for s, n in enumerate(sl)])
        nv = torch.cat([vals[s][n - ql[s]:] for s, n in enumerate(sl)])
        ns = torch.cat([slots[s][n - ql[s]:] for s, n in enumerate(sl)])
        impl.do_kv_cache_update(None, nk, nv, kv, ns)
        md = Gfx906FAMetadata(num_actual_tokens=sum(ql), max_query_len=max(ql), max_seq_len=max(sl),
                              query_start_loc=qsl, seq_lens=torch.tensor(sl, dtype=torch.int32, device=DEV),
                              block_table=btt, slot_mapping=ns)
        out = torch.empty((sum(ql), Hq * D), dtype=torch.float16, device=DEV)
        impl.forward(None, q, nk, nv, kv, md, output=out)
        outs[cd] = out
    torch.cuda.synchronize()
    (kf, vf), (kq, vq) = q8_planes(caches["auto"], Hkv, D), q8_planes(caches["q8_0"], Hkv, D)
    assert torch.equal(kf, kq) and torch.equal(vf, vq)
    assert torch.equal(outs["auto"], outs["q8_0"])
    planar = torch.stack([kq, vq], 1).cpu().numpy()
    kh, vh = O.planar_dequant(planar)
    ref = O.paged_attention_ref(q.float().cpu().numpy(), kh, vh, bt, np.asarray(sl, np.int32),
                                qsl.cpu().numpy(), 1 / math.sqrt(D))
    assert_close(outs["q8_0"].float().cpu().numpy().reshape(-1, Hq, D), ref, extra=2.0 ** -11)


# ---------------------------------------------------------------------------
# Full-size configurations: sampled-row parity + permutation invariance
# ---------------------------------------------------------------------------
def _permuted_copy(b, seed=99):
    """Same logical cache with its pages shuffled and the table remapped:
    the output must be bit-identical."""
    rng = np.random.default_rng(seed)
    perm = torch.from_numpy(rng.permutation(b.num_blocks)).to(DEV)
    inv = torch.argsort(perm)
    cache2 = b.kv_cache[perm]                       # new page i holds old page perm[i]
    bt = b.block_table.long()
    bt2 = torch.where(bt >= 0, inv[bt.clamp(min=0)], bt).to(torch.int32)
    return cache2, bt2


def _check_permutation_invariance(b, out, name):
    announce(f"{name} permutation invariance")
    cache2, bt2 = _permuted_copy(b)
    out2 = gfx906_fa.paged_attention(b.query, cache2[:, 0], cache2[:, 1], bt2, b.seq_lens_t, b.qsl_t,
                                     b.max_query_len, b.max_seq_len, b.scale, out_dtype=out.dtype)
    torch.cuda.synchronize()
    assert torch.equal(out, out2)
    del cache2


@pytest.mark.parametrize("name", ["cfg2", "cfg5"])
def test_full_size_decode_configs(name):
    """cfg2 (32 decode tokens) and cfg5 at 6/1 (8 x 5 verify tokens): every
    query token, every head, against the oracle."""
    need_gpu()
    b = W.build_cfg(name, device=DEV)
    out = _run_and_check(b, rows=list(range(b.num_tokens)))
    _check_permutation_invariance(b, out, name)


def test_full_size_verify_cfg5_48_8():
    """cfg5 rerun at the full 48/8 head shape: 8 x (131072 + 5) cached tokens,
    2.28 GB of Q8 K+V, 5 tokens x 6 q-heads = 30 packed rows per sequence and
    kv-head (the two-row-group decode class).  Every verify token of three
    sequences (first, middle, last), all 48 heads - so all 8 kv-heads -
    against the oracle; the whole output is invariant under a page
    permutation.  Shape: the reference's TP-8 deployment
    (tests/test_fa_mixed_batch.py:36-37) unsharded, verifying 1 + 4 n-gram
    draft tokens (scripts/start_vllm_fa_ngram.sh:35-39)."""
    need_gpu()
    b = W.build_cfg("cfg5", device=DEV, heads=(48, 8))
    qsl = b.qsl
    rows = [t for s in (0, 3, 7) for t in range(int(qsl[s]), int(qsl[s + 1]))]
    out = _run_and_check(b, rows=rows)
    _check_permutation_invariance(b, out, "cfg5 48/8")


def test_full_size_verify_ngram_k5():
    """The reference's n-gram verify step at full size: 8 x (131072 + 6)
    cached tokens at 6/1, 6 tokens x 6 q-heads = 36 packed rows per
    sequence (the 48-row decode class, each segment split over about 64
    workgroups).  Every verify token of every sequence against the oracle;
    the whole output is invariant under a page permutation
    (scripts/start_vllm_fa_ngram.sh:35-39)."""
    need_gpu()
    b = W.build_cfg("cfg5k6", device=DEV)
    info = gfx906_fa.plan_info(b.num_seqs, b.num_tokens, b.Hq, b.Hkv, b.max_query_len, b.max_seq_len)
    assert (info["decode_classes"], info["dec_rows_max"], info["prefill"]) == (1, 48, 0)
    out = _run_and_check(b, rows=list(range(b.num_tokens)))
    _check_permutation_invariance(b, out, "cfg5k6")


def test_full_size_prefill_cfg3():
    """cfg3, 32K causal prefill at 48/8: one query token per 8 row tiles of
    256 packed rows (every 341st token), the first and last tokens and the
    sub-page edges, every head."""
    need_gpu()
    b = W.build_cfg("cfg3", device=DEV)
    T = b.num_tokens
    rng = np.random.default_rng(3)
    sample = sorted(set(range(0, T, 341)) | {0, 1, 15, 16, 17, 63, 64, 4097, T // 2, T - 2, T - 1}
                    | set(rng.integers(0, T, 8).tolist()))
    _run_and_check(b, out_dtype=torch.float32, rows=sample)


def test_full_size_mixed_cfg4():
    """cfg4: twelve tokens of each 2048-token chunk (first and last
    included) and every fourth of the 60 decode sequences, every head."""
    need_gpu()
    b = W.build_cfg("cfg4", device=DEV)
    qsl = b.qsl
    sample = []
    for c in range(4):
        sample += np.linspace(int(qsl[c]), int(qsl[c + 1]) - 1, 12).astype(int).tolist()
    sample += [int(qsl[4 + i]) for i in range(0, 60, 4)] + [int(qsl[63])]
    _run_and_check(b, rows=sorted(set(sample)))


def test_seed_sweep_error_margin():
    """20 seeds of N(0,1) inputs: short causal prefills (fp16 and bf16, GQA
    4:1 and 6:1, a first row that sees one key) and decode batches, each
    whole output against the oracle at the north-star tolerance (max-abs
    2e-3 for fp32 output).  The worst max-abs error over the sweep is
    written to $GFA_SEED_SWEEP_OUT (JSON) when that is set."""
    need_gpu()
    worst = {}
    for seed in range(20):
        rng = np.random.default_rng(500 + seed)
        dt = "bf16" if seed % 2 else "f16"
        hq, hkv = ((8, 2), (48, 8), (6, 1), (32, 8))[seed % 4]
        L = int(rng.integers(150, 700))
        cases = {
            "prefill": W.build_batch([L], [L], hq, hkv, dtype=dt, seed=600 + seed),
            "chunk": W.build_batch([L + 300, 40], [L, 40], hq, hkv, dtype=dt, seed=700 + seed),
            "decode": W.build_batch(rng.integers(1, 3000, 8).tolist(), [1] * 8, hq, hkv, dtype=dt,
                                    seed=800 + seed),
        }
        for kind, b in cases.items():
            announce(f"seed sweep {seed} {kind} {dt} {hq}/{hkv}")
            out = W.attention(b, out_dtype=torch.float32)
            torch.cuda.synchronize()
            ref = batch_oracle(b)
            got = to_np_f32(out)
            err = float(np.abs(got - ref).max())
            if err > worst.get(kind, (0.0,))[0]:
                worst[kind] = (err, seed, dt, f"{hq}/{hkv}")
            assert_close(got, ref)
    if os.environ.get("GFA_SEED_SWEEP_OUT"):
        import json
        with open(os.environ["GFA_SEED_SWEEP_OUT"], "w") as f:
            json.dump({k: {"max_abs": v[0], "seed": v[1], "dtype": v[2], "heads": v[3]}
                       for k, v in worst.items()}, f, indent=1)


def test_decode_many_short_sequences():
    """700 decode sequences of 1..400 tokens (several per workgroup range,
    many segments shorter than a sub-page) plus a few long ones that split."""
    need_gpu()
    rng = np.random.default_rng(21)
    sl = rng.integers(1, 401, 700).tolist() + [9000, 17, 30000]
    b = W.build_batch(sl, [1] * len(sl), 16, 4, seed=21)
    _run_and_check(b)


SHORT_SPLIT = [
    # seq_lens, Hq, Hkv: contexts of at most 1024 keys, yet more decode
    # workgroups than segments, so segments are split and merged
    ("8 x 1000, 8/1", [1000] * 8, 8, 1),                       # per-row merge launch
    ("16 mixed, 48/8", [1024, 700, 33, 512] * 4, 48, 8),       # per-segment merge launch
    ("32 x 1000, 48/8", [1000] * 32, 48, 8),                   # per-segment merge launch
]


@pytest.mark.parametrize("case", SHORT_SPLIT, ids=[c[0] for c in SHORT_SPLIT])
def test_decode_short_contexts_split(case):
    """Decode batches whose contexts are all short (at most 1024 keys: the
    merge of split segments then runs one workgroup per segment when the
    resident workgroups are few per segment) but long enough that the
    stream-K plan splits segments: the plan's workgroup count (header word 1
    of the decode workspace) exceeds the segments, and the output matches
    the oracle."""
    need_gpu()
    name, sl, hq, hkv = case
    announce(f"decode short contexts split {name}")
    b = W.build_batch(sl, [1] * len(sl), hq, hkv, seed=31 + len(sl))
    kp, vp = b.planes()
    ws = gfx906_fa.new_workspace(gfx906_fa.workspace_size(b.num_seqs, b.num_tokens, b.Hq, b.Hkv, b.max_query_len,
                                                          b.max_seq_len), b.device)
    out = gfx906_fa.paged_attention(b.query, kp, vp, b.block_table, b.seq_lens_t, b.qsl_t, b.max_query_len,
                                    b.max_seq_len, b.scale, workspace=ws, out_dtype=torch.float32)
    torch.cuda.synchronize()
    u, nwg = ws[:16].view(torch.int64).cpu().tolist()
    assert nwg > len(sl) * hkv, (u, nwg)
    assert_close(to_np_f32(out), batch_oracle(b))


def test_verify_tiles_one_workgroup_per_cu():
    """5-token verify steps at 6/1 (30 rows per kv-head: the 32-row class in
    one row chunk) run one 8-wave workgroup per CU: a batch long enough to
    fill the device publishes exactly as many decode workgroups as the device
    has CUs (header word 1 of the decode workspace), its segments are split
    over them, and the output matches the oracle."""
    need_gpu()
    announce("verify tiles, one workgroup per CU: 8 x (16384 + 5), 6/1")
    b = W.build_batch([16384 + 5] * 8, [5] * 8, 6, 1, seed=77)
    kp, vp = b.planes()
    ws = gfx906_fa.new_workspace(gfx906_fa.workspace_size(b.num_seqs, b.num_tokens, b.Hq, b.Hkv, b.max_query_len,
                                                          b.max_seq_len), b.device)
    out = gfx906_fa.paged_attention(b.query, kp, vp, b.block_table, b.seq_lens_t, b.qsl_t, b.max_query_len,
                                    b.max_seq_len, b.scale, workspace=ws, out_dtype=torch.float32)
    torch.cuda.synchronize()
    u, nwg = ws[:16].view(torch.int64).cpu().tolist()
    cus = torch.cuda.get_device_properties(b.device).multi_processor_count
    assert u == 8 * ((16384 + 5 + 15) // 16) and nwg == cus, (u, nwg, cus)
    assert_close(to_np_f32(out), batch_oracle(b))


@pytest.mark.parametrize("nseq", [63, 64, 65])
def test_decode_batch_size_boundary(nseq):
    """Batches on both sides of 64 sequences (the decode kernel locates its
    segment from one per-lane metadata load up to 64, and scans the
    sequences beyond): decodes and 5-token verifies of 1..2500 tokens with
    prefill chunks (no decode work) and empty queries interleaved, so
    segments without decode sub-pages sit between split ones."""
    need_gpu()
    rng = np.random.default_rng(40 + nseq)
    kinds = rng.integers(0, 10, nseq)
    ql = [0 if k == 0 else (70 if k == 1 else (5 if k < 5 else 1)) for k in kinds]
    sl = [q + int(c) for q, c in zip(ql, rng.integers(1, 2500, nseq))]
    b = W.build_batch(sl, ql, 12, 2, seed=40 + nseq)
    _run_and_check(b)


def test_mixed_many_chunks():
    """Varlen mix of 40 prefill chunks (n_q 2..300, causal within each, prior
    context 0..3000) and 100 decode sequences in one call."""
    need_gpu()
    rng = np.random.default_rng(22)
    ql = rng.integers(2, 301, 40).tolist() + [1] * 100
    sl = [q + int(c) for q, c in zip(ql, rng.integers(0, 3001, len(ql)))]
    b = W.build_batch(sl, ql, 12, 3, seed=22)
    _run_and_check(b)


def test_forward_paged_returns_flat_fp32_and_logs(tmp_path, monkeypatch):
    """gfx906_fa_paged.forward_paged with no ``out`` returns what the
    reference's dispatcher returns, ``[num_tokens, Hq*D]`` fp32
    (extension/gfx906_fa_paged.py:197-465), for a mixed decode + chunked
    prefill batch; with GFX906_FA_FWD_DEBUG on, the call is logged before the
    launch and OK after it."""
    need_gpu()
    import gfx906_fa_paged as P
    monkeypatch.setattr(P, "_DBG", True)
    monkeypatch.setattr(P, "_DBG_DIR", str(tmp_path))
    announce("forward_paged flat fp32 + debug log")
    b = W.build_batch([700, 33, 1500], [1, 33, 200], 8, 2, seed=21)
    kp, vp = b.planes()
    res = P.forward_paged(b.query, kp, vp, b.block_table, b.seq_lens_t, b.qsl_t, b.max_query_len,
                          b.max_seq_len, b.scale)
    torch.cuda.synchronize()
    assert res.dtype == torch.float32 and tuple(res.shape) == (b.num_tokens, b.Hq * b.D)
    assert_close(res.view(b.num_tokens, b.Hq, b.D).cpu().numpy(), batch_oracle(b))
    lines = (tmp_path / f"fwd-{os.getpid()}.log").read_text().splitlines()
    assert len(lines) == 2
    assert "forward_paged VARLEN: num_tokens=234 Hq=8 Hkv=2" in lines[0]
    assert "forward_paged OK: out=(234, 8, 128)" in lines[1]
