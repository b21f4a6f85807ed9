"""CPU oracle for the Q8_0 paged-attention hot path.

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this module, and only as the
checker.  The product path (``gfx906_fa``, ``gfx906_fa_paged``,
``gfx906_fa_backend``) never imports it and fails loudly when the HIP library
is missing.

Each function restates the reference algorithm in numpy and cites the
reference file:line it follows (paths relative to the reference checkout).

Pinning (what checks each function beyond restating it):

* ``quantize_q8_0_blocks`` - closed form of ``extension/gfx906_fa_quant.cu:45-85``.
  Pinned by: the reference test's own float64 oracle
  (``tests/test_quant.py:29-52``) agreeing to <= 1 LSB on < 1 % of bytes;
  known answers (all-zero block, exact .5 ties -> even, +-amax -> +-127,
  power-of-two blocks); an independent C restatement (``oracle/q8_ref.c``)
  agreeing byte for byte; and, on the GPU box, the reference's own quant
  kernel compiled from its sources (``oracle/Makefile`` -> ``oracle/_ref``).
* ``reshape_and_cache_q8_aos`` - ``extension/gfx906_fa_quant.cu:150-200``.
  Pinned by slot arithmetic invariants (``tests/test_quant.py:80-149``):
  written rows equal the dense quantizer, untouched bytes stay, slot < 0 skips.
* ``gather_paged_kv_q8_aos`` - ``extension/gfx906_fa_gather.cu:190-357``
  (v2, the default).  Pinned by a brute-force per-token loop that follows
  ``tests/test_gather.py:15-38`` (``_ref_gather``) on tiny inputs.
* ``dequantize_q8_0_rows`` - ``tests/test_q8_roundtrip.py:21-36``.
  Pinned by dequant(quant(x)) error <= d/2 per element and exactness on
  integer-valued blocks.
* ``paged_attention_ref`` - textbook softmax(scale q K^T + causal) V over the
  dequantized cache, causal rule of ``extension/gfx906_fa_paged.py:288-295`` /
  ``kernel/fattn-q8.cuh:646-653``, GQA map of ``kernel/fattn-q8.cuh:898-901``.
  Pinned by: torch SDPA (math backend, float64) on the same dequantized
  inputs, a single visible key giving the V row, uniform scores giving the
  mean of V, invariance to block_table permutation.  Its per-kv-head core
  ``attention_rows_ref`` (explicit per-row key bounds, used directly by the
  GPU tests' sampled-row checks) is pinned through it by the same checks.
* ``flat_attention_ref`` - the contiguous path of the op module's
  ``forward`` (``extension/gfx906_fa.cpp:120-265``): dequantized K, exact
  fp16 V, kv_max cutoff and inline causal bound.  Pinned by: torch SDPA
  (math backend, float64) with the equivalent boolean mask, a single visible
  key giving the V row, and agreement with ``paged_attention_ref`` on the
  same dequantized values laid out as pages.
* ``planar_*`` - the MI355X page layouts of this build (not reference
  formats); pinned by round trips against the AoS / fp16 rows (each
  position map a bijection onto its sub-page).
* ``rope_ref`` - vLLM's rotary embedding (third-party, absent here; the
  reference's hook is ``extension/gfx906_fa_backend.py:444-445``).  Pinned
  by: an independent torch CPU restatement of vLLM's native form (16-bit
  tensor ops) agreeing bit for bit; the complex product
  (x1 + i x2)(cos + i sin) in float64 agreeing to the dtype's rounding (fixes
  the pairing and the signs); identity at angle 0; pairwise norms kept.
"""
from __future__ import annotations

import numpy as np

QK8_0 = 32          # values per Q8_0 block  (kernel/ggml_shim.cuh:90-94)
Q8_0_BYTES = 34     # fp16 scale + 32 int8   (kernel/ggml_shim.cuh:90-94)
PAGE_TOKENS = 16    # tokens per sub-page of the planar layout
SUBPAGE_BYTES = 2176  # 16 tokens * 136 bytes


def bytes_per_row(D: int) -> int:
    """(D/32)*34 - ``extension/gfx906_fa.cpp:341``."""
    assert D % QK8_0 == 0
    return (D // QK8_0) * Q8_0_BYTES


# ---------------------------------------------------------------------------
# Q8_0 closed form
# ---------------------------------------------------------------------------
def _to_f32(x) -> np.ndarray:
    """fp16 / bf16 / fp32 input -> float32 (exact for fp16 and bf16).

    bf16 arrives as a uint16 bit pattern (numpy has no bfloat16)."""
    x = np.asarray(x)
    if x.dtype == np.float16:
        return x.astype(np.float32)
    if x.dtype == np.uint16:  # bf16 bit pattern
        return (x.astype(np.uint32) << 16).view(np.float32)
    if x.dtype == np.float32:
        return x
    raise TypeError(f"unsupported input dtype {x.dtype}")


def _rint_to_int8_sat(v: np.ndarray) -> np.ndarray:
    """``(int)rintf(v)`` as the AMD ``v_cvt_i32_f32`` does it (saturating,
    NaN -> 0), then the clamp to [-128, 127] of
    ``extension/gfx906_fa_quant.cu:69-73``."""
    r = np.rint(v)  # round half to even
    r = np.where(np.isnan(r), 0.0, r)
    r = np.clip(r, -128.0, 127.0)
    return r.astype(np.int8)


def quantize_q8_0_blocks(x) -> tuple[np.ndarray, np.ndarray]:
    """Q8_0 closed form of ``extension/gfx906_fa_quant.cu:51-84``.

    x: [..., D] fp16 / bf16 (uint16 bits) / fp32.  Returns
    (q int8 [..., D], d float16 [..., D/32]).

      amax = max|x|               (fmaxf tree, order independent)
      d    = fp32(amax / 127.0f)  (IEEE single division)
      id   = d > 0 ? fp32(1.0f / d) : 0
      q    = clamp(rint(fp32(x * id)), -128, 127)
      scale stored as fp16_rne(d)
    """
    xf = _to_f32(x)
    D = xf.shape[-1]
    assert D % QK8_0 == 0
    blk = xf.reshape(*xf.shape[:-1], D // QK8_0, QK8_0)
    with np.errstate(all="ignore"):
        amax = np.max(np.abs(blk), axis=-1)                       # f32
        d = (amax / np.float32(127.0)).astype(np.float32)         # f32 div
        pos = d > np.float32(0.0)
        safe = np.where(pos, d, np.float32(1.0))
        idv = np.where(pos, np.float32(1.0) / safe, np.float32(0.0)).astype(np.float32)
        prod = (blk * idv[..., None]).astype(np.float32)          # f32 mul
    q = _rint_to_int8_sat(prod).reshape(xf.shape)
    with np.errstate(over="ignore"):
        dh = d.astype(np.float16)                                 # RNE
    return q, dh


def pack_q8_0_rows(q: np.ndarray, d: np.ndarray) -> np.ndarray:
    """block_q8_0 wire format: per block [fp16 d little-endian][32 x int8]
    (``extension/gfx906_fa_quant.cu:76-84``).  -> uint8 [..., D/32*34]."""
    D = q.shape[-1]
    nb = D // QK8_0
    lead = q.shape[:-1]
    out = np.empty((*lead, nb, Q8_0_BYTES), dtype=np.uint8)
    out[..., :2] = d.astype("<f2").reshape(*lead, nb, 1).view(np.uint8).reshape(*lead, nb, 2)
    out[..., 2:] = q.reshape(*lead, nb, QK8_0).view(np.uint8)
    return out.reshape(*lead, nb * Q8_0_BYTES)


def unpack_q8_0_rows(rows: np.ndarray, D: int) -> tuple[np.ndarray, np.ndarray]:
    rows = np.ascontiguousarray(rows, dtype=np.uint8)
    nb = D // QK8_0
    lead = rows.shape[:-1]
    r = rows.reshape(*lead, nb, Q8_0_BYTES)
    d = np.ascontiguousarray(r[..., :2]).view("<f2").reshape(*lead, nb)
    q = np.ascontiguousarray(r[..., 2:]).view(np.int8).reshape(*lead, D)
    return q, d


def quantize_q8_0_rows(x) -> np.ndarray:
    """Dense quantize (``extension/gfx906_fa_quant.cu:100-129``):
    [..., D] -> uint8 [..., D/32*34]."""
    q, d = quantize_q8_0_blocks(x)
    return pack_q8_0_rows(q, d)


def dequantize_blocks(q: np.ndarray, d: np.ndarray) -> np.ndarray:
    """x_hat = float(fp16 d) * float(int8 q)  (``tests/test_q8_roundtrip.py:21-36``)."""
    D = q.shape[-1]
    qb = q.astype(np.float32).reshape(q.shape[:-1] + (D // QK8_0, QK8_0))
    return (qb * d.astype(np.float32)[..., None]).astype(np.float32).reshape(q.shape[:-1] + (D,))


def dequantize_q8_0_rows(rows: np.ndarray, D: int) -> np.ndarray:
    q, d = unpack_q8_0_rows(rows, D)
    return dequantize_blocks(q, d)


def ref_quantize_f64(x) -> np.ndarray:
    """The reference test's own oracle (``tests/test_quant.py:29-52``):
    d and 1/d in float64, torch.round (half to even), clamp.  Used only to
    cross-check ``quantize_q8_0_rows`` within that test's tolerance."""
    xf = _to_f32(x).astype(np.float64)
    D = xf.shape[-1]
    blk = xf.reshape(-1, D // QK8_0, QK8_0)
    amax = np.max(np.abs(blk), axis=-1)
    d = amax / 127.0
    idv = np.where(d > 0, 1.0 / np.where(d > 0, d, 1.0), 0.0)
    q = np.clip(np.rint(blk * idv[..., None]), -128, 127).astype(np.int8)
    out = np.empty((blk.shape[0], D // QK8_0, Q8_0_BYTES), dtype=np.uint8)
    out[..., :2] = d.astype(np.float16).reshape(-1, D // QK8_0, 1).view(np.uint8).reshape(-1, D // QK8_0, 2)
    out[..., 2:] = q.view(np.uint8)
    return out.reshape(*xf.shape[:-1], D // QK8_0 * Q8_0_BYTES)


# ---------------------------------------------------------------------------
# Reference AoS cache write and gather
# ---------------------------------------------------------------------------
def reshape_and_cache_q8_aos(key, slot_mapping: np.ndarray, cache: np.ndarray) -> None:
    """In-place write of ``extension/gfx906_fa_quant.cu:150-200``.

    key: [T, Hkv, D]; slot_mapping: int64 [T]; cache: uint8
    [NB, bs, Hkv, bpr] (any numpy view; strides are honoured).
    slot < 0 -> token skipped; every other byte untouched."""
    T, Hkv, D = np.asarray(key).shape
    bs = cache.shape[1]
    rows = quantize_q8_0_rows(key)  # [T, Hkv, bpr]
    for t in range(T):
        s = int(slot_mapping[t])
        if s < 0:
            continue
        cache[s // bs, s % bs, :, :] = rows[t]


def gather_paged_kv_q8_aos(key_cache_q8: np.ndarray, value_cache: np.ndarray,
                           block_table: np.ndarray, seq_lens: np.ndarray, Sk: int,
                           k_out: np.ndarray | None = None,
                           v_out: np.ndarray | None = None):
    """``extension/gfx906_fa_gather.cu:190-357`` (v2, default) contract.

    For s, h, t < Sk:  lb = t // bs;  pb = bt[s, lb] if lb < M else -1.
    If t < seq_len[s] and pb >= 0: copy K row and V row.
    Else V row = 0 and K row untouched (caller's buffer keeps its bytes).

    value_cache may be fp16 [NB, bs, Hkv, D] (reference) or uint8 AoS
    [NB, bs, Hkv, bpr] (the Q8/Q8 variant of this build)."""
    NB, bs, Hkv, bpr = key_cache_q8.shape
    B, M = block_table.shape
    vrow = value_cache.shape[-1]
    if k_out is None:
        k_out = np.zeros((B, Hkv, Sk, bpr), dtype=np.uint8)
    if v_out is None:
        v_out = np.zeros((B, Hkv, Sk, vrow), dtype=value_cache.dtype)
    for s in range(B):
        sl = int(seq_lens[s])
        for t in range(Sk):
            lb = t // bs
            pb = int(block_table[s, lb]) if lb < M else -1
            if t < sl and pb >= 0:
                k_out[s, :, t, :] = key_cache_q8[pb, t % bs, :, :]
                v_out[s, :, t, :] = value_cache[pb, t % bs, :, :]
            else:
                v_out[s, :, t, :] = 0
    return k_out, v_out


# ---------------------------------------------------------------------------
# Planar MFMA page layout of this build (D = 128)
# ---------------------------------------------------------------------------
# Per (page, kv-head) each 16-token sub-page is 2176 bytes:
#   K plane: int8 q[t][d] at kpos(t, d), with b = d//32, g = (d%32)//8:
#              kpos = (b//2)*1024 + (4t + g)*16 + (b%2)*8 + d%8
#            fp16 d[t][b] at 2048 + (4t+b)*2
#   V plane: int8 q[t][d] at vpos(t, d), with m = d//16:
#              vpos = (m//4)*1024 + ((t//4)*16 + d%16)*16 + (m%4)*4 + t%4
#            fp16 d[t][b] at 2048 + ((t//4)*4 + b)*8 + (t%4)*2
# Each half (1024 bytes) of the int area is what one wave-wide 16-byte load
# instruction reads, fully contiguous.
def planar_kpos(t, d) -> np.ndarray:
    t = np.asarray(t)
    d = np.asarray(d)
    b, g = d // 32, (d % 32) // 8
    return (b // 2) * 1024 + (4 * t + g) * 16 + (b % 2) * 8 + d % 8


def planar_vpos(t, d) -> np.ndarray:
    t = np.asarray(t)
    d = np.asarray(d)
    m = d // 16
    return (m // 4) * 1024 + ((t // 4) * 16 + d % 16) * 16 + (m % 4) * 4 + t % 4


def planar_spos(plane: int, t, b):
    """Byte offset of fp16 scale (t, b) inside a sub-page."""
    t = np.asarray(t)
    b = np.asarray(b)
    if plane == 0:
        return 2048 + (4 * t + b) * 2
    return 2048 + ((t // 4) * 4 + b) * 8 + (t % 4) * 2


def planar_cache_shape(num_blocks: int, block_size: int, Hkv: int, D: int = 128):
    """[NB, 2, Hkv, bs/16 * 2176] uint8."""
    assert D == 128 and block_size % PAGE_TOKENS == 0
    return (num_blocks, 2, Hkv, (block_size // PAGE_TOKENS) * SUBPAGE_BYTES)


def planar_write_rows(cache: np.ndarray, plane: int, page: int, head: int, tok: int,
                      q_row: np.ndarray, d_row: np.ndarray) -> None:
    """Store one token row (q int8 [128], d fp16 [4]) into the planar cache."""
    sp, t = divmod(tok, PAGE_TOKENS)
    base = sp * SUBPAGE_BYTES
    dd = np.arange(128)
    buf = cache[page, plane, head]
    if plane == 0:
        buf[base + planar_kpos(t, dd)] = q_row.view(np.uint8)
    else:
        buf[base + planar_vpos(t, dd)] = q_row.view(np.uint8)
    sc = np.asarray(d_row, dtype="<f2").view(np.uint8).reshape(4, 2)
    for b in range(4):
        o = base + int(planar_spos(plane, t, b))
        buf[o:o + 2] = sc[b]


def planar_read_rows(cache: np.ndarray, plane: int, page: int, head: int, tok: int):
    """-> (q int8 [128], d fp16 [4]) for one token."""
    sp, t = divmod(tok, PAGE_TOKENS)
    base = sp * SUBPAGE_BYTES
    dd = np.arange(128)
    buf = cache[page, plane, head]
    if plane == 0:
        q = buf[base + planar_kpos(t, dd)].view(np.int8)
    else:
        q = buf[base + planar_vpos(t, dd)].view(np.int8)
    so = base + planar_spos(plane, t, np.arange(4))
    d = np.ascontiguousarray(np.stack([buf[so], buf[so + 1]], axis=-1)).view("<f2").reshape(4)
    return q.copy(), d.copy()


def planar_cache_write(key, value, slot_mapping: np.ndarray, cache: np.ndarray) -> None:
    """K and V of each token quantized with the Q8_0 closed form and stored
    at ``slot_mapping`` (slot < 0 skipped) - the K+V analogue of
    ``extension/gfx906_fa_quant.cu:150-200`` for the planar layout."""
    T, Hkv, D = np.asarray(key).shape
    assert D == 128
    bs = (cache.shape[3] // SUBPAGE_BYTES) * PAGE_TOKENS
    qk, dk = quantize_q8_0_blocks(key)
    qv, dv = quantize_q8_0_blocks(value)
    for t in range(T):
        s = int(slot_mapping[t])
        if s < 0:
            continue
        page, off = divmod(s, bs)
        for h in range(Hkv):
            planar_write_rows(cache, 0, page, h, off, qk[t, h], dk[t, h])
            planar_write_rows(cache, 1, page, h, off, qv[t, h], dv[t, h])


def planar_to_aos(cache: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Planar cache -> (K AoS [NB, bs, Hkv, 136], V AoS [NB, bs, Hkv, 136]).

    The position maps above are products of index splits, so a sub-page
    unpacks by reshape + transpose:
      K ints  [b//2][t][g][b%2][d%8] -> [t][b][g][d%8]    (d = 32b + 8g + d%8)
      K scales [t][b]
      V ints  [m//4][t//4][d%16][m%4][t%4] -> [t//4][t%4][m][d%16]  (d = 16m + d%16)
      V scales [t//4][b][t%4] -> [t//4][t%4][b]"""
    NB, _, Hkv, nbytes = cache.shape
    nsp = nbytes // SUBPAGE_BYTES
    bs = nsp * PAGE_TOKENS
    sub = np.ascontiguousarray(cache).reshape(NB, 2, Hkv, nsp, SUBPAGE_BYTES)
    ints, scales = sub[..., :2048], sub[..., 2048:]
    lead = (NB, Hkv, nsp)
    kq = ints[:, 0].reshape(*lead, 2, 16, 4, 2, 8).transpose(0, 1, 2, 4, 3, 6, 5, 7)  # t, bh, bl, g, e
    kq = kq.reshape(*lead, 16, 4, 32)
    ks = scales[:, 0].reshape(*lead, 16, 4, 2)
    vq = ints[:, 1].reshape(*lead, 2, 4, 16, 4, 4).transpose(0, 1, 2, 4, 7, 3, 6, 5)  # tq, tl, mh, ml, dl
    vq = vq.reshape(*lead, 16, 4, 32)
    vs = scales[:, 1][..., :128].reshape(*lead, 4, 4, 4, 2).transpose(0, 1, 2, 3, 5, 4, 6)  # tq, tl, b
    vs = vs.reshape(*lead, 16, 4, 2)
    out = []
    for q, sc in ((kq, ks), (vq, vs)):
        rows = np.concatenate([sc, q], axis=-1)                  # [NB, Hkv, nsp, 16, 4, 34]
        rows = rows.reshape(NB, Hkv, bs, 136).transpose(0, 2, 1, 3)
        out.append(np.ascontiguousarray(rows))
    return out[0], out[1]


def planar_dequant(cache: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Planar cache -> dequantized (K, V) float32 [NB, bs, Hkv, 128]."""
    ko, vo = planar_to_aos(cache)
    return dequantize_q8_0_rows(ko, 128), dequantize_q8_0_rows(vo, 128)


# ---------------------------------------------------------------------------
# Attention reference
# ---------------------------------------------------------------------------
def attention_rows_ref(q: np.ndarray, K: np.ndarray, V: np.ndarray, lim: np.ndarray,
                       scale: float) -> np.ndarray:
    """The softmax core of ``paged_attention_ref`` for the query heads of one
    kv-head: q [n, G, D] (n query rows of G heads each), K / V [L, D] that
    kv-head's dequantized keys and values in position order, lim [n]: row i
    sees keys k <= lim[i].  -> float64 [n, G, D]; a row with no visible key
    (lim < 0) outputs 0."""
    q = np.asarray(q, np.float64)
    K = np.asarray(K, np.float64)
    V = np.asarray(V, np.float64)
    lim = np.asarray(lim, np.int64)
    pos = np.arange(K.shape[0])
    mask = pos[None, :] <= lim[:, None]              # [n, L]
    n, G, D = q.shape
    sc = (q.reshape(n * G, D) @ K.T).reshape(n, G, -1) * scale
    sc = np.where(mask[:, None, :], sc, -np.inf)
    m = np.max(sc, axis=-1, keepdims=True) if sc.shape[-1] else np.zeros(sc.shape[:-1] + (1,))
    m = np.where(np.isfinite(m), m, 0.0)
    p = np.exp(sc - m)
    p = np.where(mask[:, None, :], p, 0.0)
    l = p.sum(-1, keepdims=True)
    o = (p.reshape(n * G, -1) @ V).reshape(n, G, V.shape[1])
    return np.where(l > 0, o / np.where(l > 0, l, 1.0), 0.0)


def paged_attention_ref(query: np.ndarray, k_hat: np.ndarray, v_hat: np.ndarray,
                        block_table: np.ndarray, seq_lens: np.ndarray,
                        query_start_loc: np.ndarray, scale: float) -> np.ndarray:
    """Dequantize-then-float64 softmax attention over a paged cache.

    query: [T, Hq, D]; k_hat / v_hat: dequantized [NB, bs, Hkv, D];
    block_table [B, M]; seq_lens [B]; query_start_loc [B+1].
    Row j of sequence s (0 <= j < n_q) sees keys k <= seq_lens[s] - n_q + j
    (``extension/gfx906_fa_paged.py:288-295``, ``kernel/fattn-q8.cuh:646-653``);
    q-head h reads kv-head h // (Hq/Hkv) (``kernel/fattn-q8.cuh:898-901``).
    A row with no visible key outputs 0 (``seq_len = 0``; the reference
    divides by zero there)."""
    T, Hq, D = query.shape
    NB, bs, Hkv, _ = k_hat.shape
    G = Hq // Hkv
    out = np.zeros((T, Hq, D), dtype=np.float64)
    B = len(seq_lens)
    for s in range(B):
        q0, q1 = int(query_start_loc[s]), int(query_start_loc[s + 1])
        nq = q1 - q0
        sl = int(seq_lens[s])
        if nq <= 0 or sl <= 0:
            continue
        pos = np.arange(sl)
        pages = block_table[s, pos // bs].astype(np.int64)
        K = k_hat[pages, pos % bs]                       # [sl, Hkv, D]
        V = v_hat[pages, pos % bs]
        lim = sl - nq + np.arange(nq)                    # [nq]
        for h in range(Hkv):
            out[q0:q1, h * G:(h + 1) * G, :] = attention_rows_ref(
                query[q0:q1, h * G:(h + 1) * G, :], K[:, h, :], V[:, h, :], lim, scale)
    return out


def flat_attention_ref(q: np.ndarray, k_aos: np.ndarray, v: np.ndarray, scale: float,
                       kv_max=None, q_abs_offset=None, mask=None) -> np.ndarray:
    """Contiguous attention of the op module's ``forward``
    (``extension/gfx906_fa.cpp:120-265``; kernel ``kernel/fattn-q8.cuh:835-1087``)
    over dequantized K and exact fp16 V, float64 softmax.

    q [B, Hq, Sq, D]; k_aos uint8 [B, Hkv, Skv, D/32*34]; v [B, Hkv, Skv, D]
    -> [B, Hq, Sq, D].  Row j of batch b sees key k when k < kv_max[b] (all
    Skv keys without kv_max; ``extension/gfx906_fa.cpp:189-212``) and, with
    q_abs_offset, k <= q_abs_offset[b] + j (``kernel/fattn-q8.cuh:646-653``).
    q-head h reads kv-head h // (Hq/Hkv) (``kernel/fattn-q8.cuh:898-901``).
    mask [B, Sq, >= Skv]: added to the scaled scores
    (``kernel/fattn-q8.cuh:643-644``).  A row with no visible key outputs 0."""
    B, Hq, Sq, D = q.shape
    Hkv, Skv = v.shape[1], v.shape[2]
    G = Hq // Hkv
    K = dequantize_q8_0_rows(k_aos, D).astype(np.float64)   # [B, Hkv, Skv, D]
    V = np.asarray(v, dtype=np.float64)
    out = np.zeros((B, Hq, Sq, D), dtype=np.float64)
    pos = np.arange(Skv)
    for b in range(B):
        cut = Skv if kv_max is None else min(max(int(kv_max[b]), 0), Skv)
        vis = np.broadcast_to(pos[None, :] < cut, (Sq, Skv))
        if q_abs_offset is not None:
            vis = vis & (pos[None, :] <= int(q_abs_offset[b]) + np.arange(Sq)[:, None])
        for h in range(Hkv):
            qh = q[b, h * G:(h + 1) * G].astype(np.float64)           # [G, Sq, D]
            sc = np.einsum("gjd,kd->gjk", qh, K[b, h]) * scale
            if mask is not None:
                sc = sc + np.asarray(mask[b], dtype=np.float64)[None, :, :Skv]
            vis2 = vis[None] & (sc > -np.inf)
            sc = np.where(vis2, sc, -np.inf)
            m = np.max(sc, axis=-1, keepdims=True)
            m = np.where(np.isfinite(m), m, 0.0)
            p = np.where(vis2, np.exp(sc - m), 0.0)
            l = p.sum(-1, keepdims=True)
            o = np.einsum("gjk,kd->gjd", p, V[b, h])
            out[b, h * G:(h + 1) * G] = np.where(l > 0, o / np.where(l > 0, l, 1.0), 0.0)
    return out


def planar_v16_pos(t, d) -> np.ndarray:
    """Byte offset of fp16 V element (t, d) inside a 4096-byte planar fp16
    sub-page (the layout of the flat entry's repacked V)."""
    t = np.asarray(t)
    d = np.asarray(d)
    return 2048 * (d // 64) + 32 * (16 * (t // 4) + d % 16) + 8 * ((d // 16) % 4) + 2 * (t % 4)


# ---------------------------------------------------------------------------
# Seeded workload generators (CPU seeds; same inputs on every machine)
# ---------------------------------------------------------------------------
def make_block_table(rng: np.random.Generator, seq_lens, block_size: int,
                     num_blocks: int | None = None, pad_cols: int = 0):
    """Random permutation of a shared page pool; returns (block_table int32
    [B, M], num_blocks).  Unused columns are -1."""
    seq_lens = [int(x) for x in seq_lens]
    need = [(sl + block_size - 1) // block_size for sl in seq_lens]
    total = sum(need)
    if num_blocks is None:
        num_blocks = total + 1
    M = max(max(need) if need else 1, 1) + pad_cols
    perm = rng.permutation(num_blocks)[:total]
    bt = np.full((len(seq_lens), M), -1, dtype=np.int32)
    c = 0
    for s, n in enumerate(need):
        bt[s, :n] = perm[c:c + n]
        c += n
    return bt, num_blocks


def slots_for(block_table: np.ndarray, s: int, positions, block_size: int) -> np.ndarray:
    positions = np.asarray(positions, dtype=np.int64)
    return block_table[s, positions // block_size].astype(np.int64) * block_size + positions % block_size


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bit pattern (uint16), round to nearest even."""
    u = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return r


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


# ---------------------------------------------------------------------------
# Rotary embedding (the fused rope + cache write)
# ---------------------------------------------------------------------------
# The reference declares no fused rope + KV write (its backend returns False
# from fused_rope_kvcache_supported, extension/gfx906_fa_backend.py:444-445);
# the rotary arithmetic belongs to vLLM (0.19.1, pinned by the reference's
# README.md:29 and docker/Dockerfile:24; not vendored, not installed here).
# Its published form (RotaryEmbedding.forward_native / _apply_rotary_emb_torch,
# and the device kernel apply_token_rotary_embedding) is restated below:
#   cos, sin = cos_sin_cache[pos].chunk(2); cos, sin -> x.dtype
#   neox:  x1, x2 = x[..., :rot/2], x[..., rot/2:rot]
#   gptj:  x1, x2 = x[..., 0:rot:2], x[..., 1:rot:2]
#   o1 = x1*cos - x2*sin;  o2 = x2*cos + x1*sin     (each op in x.dtype)
# A 16-bit tensor op is computed in float32 and rounded once to the tensor's
# dtype, so every product, difference and sum is rounded here too.
def _round_model(x32: np.ndarray, bf16: bool) -> np.ndarray:
    """float32 -> model dtype (fp16 or bf16, RNE) -> float32."""
    x32 = np.asarray(x32, dtype=np.float32)
    if bf16:
        return bf16_bits_to_f32(f32_to_bf16_bits(x32))
    return x32.astype(np.float16).astype(np.float32)


def rope_cos_sin_cache(max_position: int, rot_dim: int, base: float = 10000.0) -> np.ndarray:
    """float32 [max_position, rot_dim]: cos | sin of position * base^(-2i/rot)
    (vLLM's RotaryEmbedding._compute_cos_sin_cache)."""
    inv = 1.0 / (base ** (np.arange(0, rot_dim, 2, dtype=np.float32) / rot_dim))
    f = np.outer(np.arange(max_position, dtype=np.float32), inv.astype(np.float32)).astype(np.float32)
    return np.concatenate([np.cos(f), np.sin(f)], axis=-1).astype(np.float32)


def rope_ref(x, positions: np.ndarray, cos_sin, rot_dim: int, is_neox: bool):
    """Rotary embedding of x [T, H, D] (fp16, or bf16 as uint16 bits) at
    positions [T]; returns the same dtype.  cos_sin [P, >= rot_dim] in
    float32, fp16 or bf16 bits (converted to x's dtype first).  Rows whose
    position is outside [0, P) are returned unchanged."""
    x = np.asarray(x)
    bf16 = x.dtype == np.uint16
    xf = _to_f32(x).copy()                           # [T, H, D]
    cs = _to_f32(np.asarray(cos_sin))
    P = cs.shape[0]
    half = rot_dim // 2
    pos = np.asarray(positions, dtype=np.int64)
    ok = (pos >= 0) & (pos < P)
    p = np.where(ok, pos, 0)
    c = _round_model(cs[p, :half], bf16)[:, None, :]          # [T, 1, half]
    s = _round_model(cs[p, half:rot_dim], bf16)[:, None, :]
    r = lambda a: _round_model(a, bf16)                         # noqa: E731
    if is_neox:
        x1, x2 = xf[..., :half], xf[..., half:rot_dim]
    else:
        x1, x2 = xf[..., 0:rot_dim:2], xf[..., 1:rot_dim:2]
    o1 = r(r(x1 * c) - r(x2 * s))
    o2 = r(r(x2 * c) + r(x1 * s))
    out = xf.copy()
    if is_neox:
        out[..., :half], out[..., half:rot_dim] = o1, o2
    else:
        out[..., 0:rot_dim:2], out[..., 1:rot_dim:2] = o1, o2
    out[~ok] = xf[~ok]
    if bf16:
        return f32_to_bf16_bits(out)
    return out.astype(np.float16)
