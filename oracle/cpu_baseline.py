"""CPU baseline: the reference's PyTorch CPU attention path, restated.

TEST / MEASUREMENT INFRASTRUCTURE ONLY (the ``cpu_baseline`` leg of
``bench.py``); never part of the product path.

What is timed, per sequence (streaming, so fp32 K/V never materialise for the
whole batch):
  1. gather the sequence's Q8_0 rows from the paged AoS cache by block table
     (torch fancy indexing, as ``extension/gfx906_fa_paged.py:148-194``);
  2. dequantize: float(fp16 d) * int8 q (``tests/test_q8_roundtrip.py:21-36``);
  3. ``torch.nn.functional.scaled_dot_product_attention`` in fp32 with GQA
     expansion (``repeat_interleave``) and the causal rule "row j sees keys
     <= seq_len - n_q + j" (``tests/test_fa_mixed_batch.py:135-160``).
The AoS caches are built (outside the timed region) from this build's planar
cache; they hold exactly the reference's block_q8_0 rows.
"""
from __future__ import annotations

import os
import time

import numpy as np
import torch

from oracle import q8_oracle as O


def aos_from_planar(cache_u8: np.ndarray):
    """-> (K AoS, V AoS) uint8 torch tensors [NB, bs, Hkv, 136]."""
    ka, va = O.planar_to_aos(cache_u8)
    return torch.from_numpy(ka), torch.from_numpy(va)


def _dequant(rows: torch.Tensor) -> torch.Tensor:
    """uint8 [..., 136] -> fp32 [..., 128]."""
    lead = rows.shape[:-1]
    r = rows.reshape(-1, 4, 34)
    d = r[:, :, :2].contiguous().view(torch.float16).float()       # [N, 4, 1]
    q = r[:, :, 2:].contiguous().view(torch.int8).float()          # [N, 4, 32]
    return (q * d).reshape(*lead, 128)


def attention_cpu(query: torch.Tensor, k_aos: torch.Tensor, v_aos: torch.Tensor,
                  block_table: np.ndarray, seq_lens: np.ndarray, q_lens: np.ndarray,
                  scale: float, seqs=None) -> torch.Tensor:
    """query fp32 [T, Hq, 128] -> fp32 [T, Hq, 128] (rows of `seqs` only)."""
    T, Hq, D = query.shape
    NB, bs, Hkv, _ = k_aos.shape
    G = Hq // Hkv
    out = torch.zeros((T, Hq, D), dtype=torch.float32)
    qsl = np.concatenate([[0], np.cumsum(q_lens)])
    for s in (range(len(seq_lens)) if seqs is None else seqs):
        sl, nq, q0 = int(seq_lens[s]), int(q_lens[s]), int(qsl[s])
        if nq == 0 or sl == 0:
            continue
        nb = (sl + bs - 1) // bs
        pages = torch.from_numpy(block_table[s, :nb].astype(np.int64))
        K = _dequant(k_aos[pages].reshape(nb * bs, Hkv, 136)[:sl])       # [sl, Hkv, D]
        V = _dequant(v_aos[pages].reshape(nb * bs, Hkv, 136)[:sl])
        K = K.permute(1, 0, 2).repeat_interleave(G, dim=0)                 # [Hq, sl, D]
        V = V.permute(1, 0, 2).repeat_interleave(G, dim=0)
        q = query[q0:q0 + nq].permute(1, 0, 2)                             # [Hq, nq, D]
        mask = None
        if nq > 1:
            mask = torch.arange(sl)[None, :] <= (sl - nq + torch.arange(nq))[:, None]
        o = torch.nn.functional.scaled_dot_product_attention(q[None], K[None], V[None],
                                                             attn_mask=None if mask is None else mask[None, None],
                                                             scale=scale)
        out[q0:q0 + nq] = o[0].permute(1, 0, 2)
    return out


def host_threads() -> int:
    """Threads the CPU baseline runs on: the CPUs this process may run on
    (its affinity mask), capped by OMP_NUM_THREADS when that is set (the
    process's share of a shared host)."""
    n = len(os.sched_getaffinity(0))
    env = os.environ.get("OMP_NUM_THREADS", "")
    if env.isdigit() and int(env) > 0:
        n = min(n, int(env))
    return max(n, 1)


def set_threads() -> int:
    n = host_threads()
    torch.set_num_threads(n)
    return torch.get_num_threads()


def time_cpu_decode(query: torch.Tensor, k_aos, v_aos, block_table, seq_lens, q_lens, scale,
                    budget_s: float = 10.0):
    """Runs whole sequences in batch order, pass after pass, until `budget_s`
    is spent (at least one sequence).  Returns (seconds, cached tokens read,
    sequences run, whole passes, threads)."""
    set_threads()
    tokens = seqs = 0
    t0 = time.perf_counter()
    while True:
        for s in range(len(seq_lens)):
            attention_cpu(query, k_aos, v_aos, block_table, seq_lens, q_lens, scale, seqs=[s])
            tokens += int(seq_lens[s])
            seqs += 1
            if time.perf_counter() - t0 >= budget_s:
                return time.perf_counter() - t0, tokens, seqs, seqs // len(seq_lens), torch.get_num_threads()


def head_kv_cpu(k_aos, v_aos, block_table: np.ndarray, seq_len: int, kv_head: int):
    """Dequantized K, V fp32 [seq_len, D] of one kv-head of one sequence."""
    bs = k_aos.shape[1]
    nb = (seq_len + bs - 1) // bs
    pages = torch.from_numpy(block_table[:nb].astype(np.int64))
    K = _dequant(k_aos[pages, :, kv_head].reshape(nb * bs, 136)[:seq_len])
    V = _dequant(v_aos[pages, :, kv_head].reshape(nb * bs, 136)[:seq_len])
    return K, V


def prefill_chunk_cpu(qh: torch.Tensor, K: torch.Tensor, V: torch.Tensor, r0: int, r1: int, seq_len: int,
                      scale: float) -> torch.Tensor:
    """Query rows [r0, r1) of a prompt of qh.shape[1] rows (G heads of one
    kv-head, qh [G, n_q, D]) over K, V [seq_len, D]: one fp32 SDPA over the
    keys up to the chunk's last row, row j seeing keys <= seq_len - n_q + j.
    -> [G, r1 - r0, D]."""
    G, nq, D = qh.shape
    kend = seq_len - nq + r1                                             # keys [0, kend)
    lim = seq_len - nq + torch.arange(r0, r1)
    mask = torch.arange(kend)[None, :] <= lim[:, None]
    o = torch.nn.functional.scaled_dot_product_attention(qh[None, :, r0:r1], K[None, None, :kend].expand(1, G, kend, D),
                                                         V[None, None, :kend].expand(1, G, kend, D),
                                                         attn_mask=mask[None, None], scale=scale)
    return o[0]


def time_cpu_prefill(query: torch.Tensor, k_aos, v_aos, block_table: np.ndarray, seq_len: int, scale: float,
                     chunk: int = 1024, budget_s: float = 10.0):
    """Causal prefill of one sequence (query rows = its last len(query)
    positions; here the whole prompt) by the reference's CPU path, q-chunked
    since a whole fp32 score matrix of a 32K prompt would not fit (206 GB at
    48 heads): kv-head by kv-head, dequantize that head's K and V
    (tests/test_q8_roundtrip.py:21-36), then for each chunk of `chunk` query
    rows one fp32 SDPA of its G query heads over the keys up to the chunk's
    last row with the causal mask "row j sees keys <= seq_len - n_q + j"
    (tests/test_fa_mixed_batch.py:135-160).  Within a head the chunks run in
    a fixed spread order (first, last, second, ...); kv-heads run until
    `budget_s` is spent (at least one chunk).  Attention cost is linear in
    heads, so the rate over the heads run is the rate of all heads.
    Returns (seconds, attention FLOP done (4*D*G*visible keys of the rows
    run), kv-heads started, chunks run, chunks per head, G, threads)."""
    thr = set_threads()
    T, Hq, D = query.shape
    NB, bs, Hkv, _ = k_aos.shape
    G = Hq // Hkv
    nq = T
    nchunks = (nq + chunk - 1) // chunk
    order = []
    lo, hi = 0, nchunks - 1
    while lo <= hi:                       # first, last, second, second-to-last, ...
        order.append(lo)
        if hi != lo:
            order.append(hi)
        lo, hi = lo + 1, hi - 1
    t0 = time.perf_counter()
    flop = 0.0
    heads = done = 0
    for h in range(Hkv):
        heads += 1
        K, V = head_kv_cpu(k_aos, v_aos, block_table, seq_len, h)
        qh = query[:, h * G:(h + 1) * G].permute(1, 0, 2)                   # [G, nq, D]
        for c in order:
            r0, r1 = c * chunk, min((c + 1) * chunk, nq)
            prefill_chunk_cpu(qh, K, V, r0, r1, seq_len, scale)
            flop += 4.0 * D * G * int((seq_len - nq + torch.arange(r0, r1) + 1).sum())
            done += 1
            if time.perf_counter() - t0 >= budget_s:
                return time.perf_counter() - t0, flop, heads, done, nchunks, G, thr
    return time.perf_counter() - t0, flop, heads, done, nchunks, G, thr
