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


def time_cpu_decode(query: torch.Tensor, k_aos, v_aos, block_table, seq_lens, q_lens, scale,
                    budget_s: float = 10.0):
    """Runs whole sequences in batch order, pass after pass, until `budget_s`
    is spent (at least one sequence).  Returns (seconds, cached tokens read,
    sequences run, whole passes, threads)."""
    torch.set_num_threads(torch.get_num_threads())
    tokens = seqs = 0
    t0 = time.perf_counter()
    while True:
        for s in range(len(seq_lens)):
            attention_cpu(query, k_aos, v_aos, block_table, seq_lens, q_lens, scale, seqs=[s])
            tokens += int(seq_lens[s])
            seqs += 1
            if time.perf_counter() - t0 >= budget_s:
                return time.perf_counter() - t0, tokens, seqs, seqs // len(seq_lens), torch.get_num_threads()
