"""Seeded synthetic workloads for the Q8_0 paged-attention path.

The five configurations of the benchmark definition (cfg1..cfg5) and a
generic builder.  Sequence lengths, block tables and slot mappings are drawn
on the CPU with ``numpy.random.default_rng(seed)`` so every machine builds
the same batch; K/V/Q values are N(0,1), drawn on the CPU for small batches
(reproducible bit for bit) or on the device from a seeded generator for the
full-size ones.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Optional

import numpy as np
import torch

import gfx906_fa

_TD = {"f16": torch.float16, "bf16": torch.bfloat16, "f32": torch.float32}


@dataclass
class Batch:
    """One attention batch over a planar Q8 KV cache (all tensors on `device`)."""
    Hq: int
    Hkv: int
    D: int
    block_size: int
    seq_lens: np.ndarray          # int32 [B] (new tokens included)
    q_lens: np.ndarray            # int32 [B]
    block_table_np: np.ndarray    # int32 [B, M]
    num_blocks: int
    dtype: str
    scale: float
    device: torch.device
    query: Optional[torch.Tensor] = None        # [T, Hq, D]
    key: Optional[torch.Tensor] = None          # [sum(seq_lens), Hkv, D] all cached tokens
    value: Optional[torch.Tensor] = None
    slot_mapping: Optional[torch.Tensor] = None  # int64 [sum(seq_lens)]
    kv_cache: Optional[torch.Tensor] = None      # uint8 [NB, 2, Hkv, bs/16*2176]
    block_table: Optional[torch.Tensor] = None
    seq_lens_t: Optional[torch.Tensor] = None
    qsl_t: Optional[torch.Tensor] = None
    meta: dict = field(default_factory=dict)

    @property
    def num_seqs(self) -> int:
        return len(self.seq_lens)

    @property
    def num_tokens(self) -> int:
        return int(self.q_lens.sum())

    @property
    def qsl(self) -> np.ndarray:
        return np.concatenate([[0], np.cumsum(self.q_lens)]).astype(np.int32)

    @property
    def max_query_len(self) -> int:
        return int(self.q_lens.max()) if len(self.q_lens) else 0

    @property
    def max_seq_len(self) -> int:
        return int(self.seq_lens.max()) if len(self.seq_lens) else 0

    def planes(self):
        return self.kv_cache[:, 0], self.kv_cache[:, 1]

    # --- algorithmic work (the roofline numerators) -------------------------
    def kv_bytes(self) -> int:
        """Q8 K+V bytes every attention pass must read: per cached token and
        kv-head 2 x 136 bytes (visible keys only, causal rows included)."""
        return int(self.seq_lens.astype(np.int64).sum()) * self.Hkv * 2 * (self.D // 32 * 34)

    def hbm_bytes(self, out_bytes_per_elem: int) -> int:
        T = self.num_tokens
        qb = {"f16": 2, "bf16": 2, "f32": 4}[self.dtype]
        bt = int(sum((int(s) + self.block_size - 1) // self.block_size for s in self.seq_lens)) * 4
        return self.kv_bytes() + T * self.Hq * self.D * (qb + out_bytes_per_elem) + bt

    def flops(self) -> float:
        """4*D*Hq*sum over query rows of visible keys (QK^T and PV)."""
        tot = 0
        for sl, nq in zip(self.seq_lens.astype(np.int64), self.q_lens.astype(np.int64)):
            # row j sees sl - nq + j + 1 keys
            tot += nq * (sl - nq) + nq * (nq + 1) // 2
        return 4.0 * self.D * self.Hq * float(tot)


def make_block_table(rng: np.random.Generator, seq_lens, block_size: int, extra_blocks: int = 1):
    need = [(int(s) + block_size - 1) // block_size for s in seq_lens]
    total = sum(need)
    num_blocks = total + extra_blocks
    perm = rng.permutation(num_blocks)[:total].astype(np.int32)
    M = max(max(need) if need else 1, 1)
    bt = np.full((len(need), M), -1, dtype=np.int32)
    c = 0
    for s, n in enumerate(need):
        bt[s, :n] = perm[c:c + n]
        c += n
    return bt, num_blocks


def build_batch(seq_lens, q_lens, Hq: int, Hkv: int, *, D: int = 128, block_size: int = 16,
                dtype: str = "f16", seed: int = 0, device="cuda", host_values: bool = True,
                write_cache: bool = True, bt_pad_cols: int = 0) -> Batch:
    """Builds a batch, fills the planar Q8 cache with the quantized K/V of
    every cached token (through the HIP cache-write kernel) and draws Q."""
    rng = np.random.default_rng(seed)
    seq_lens = np.asarray(seq_lens, dtype=np.int32)
    q_lens = np.asarray(q_lens, dtype=np.int32)
    bt, nb = make_block_table(rng, seq_lens, block_size)
    if bt_pad_cols:
        bt = np.concatenate([bt, np.full((bt.shape[0], bt_pad_cols), -1, np.int32)], axis=1)
    dev = torch.device(device)
    b = Batch(Hq=Hq, Hkv=Hkv, D=D, block_size=block_size, seq_lens=seq_lens, q_lens=q_lens,
              block_table_np=bt, num_blocks=nb, dtype=dtype, scale=1.0 / math.sqrt(D), device=dev)
    ntok = int(seq_lens.astype(np.int64).sum())
    T = b.num_tokens
    td = _TD[dtype]
    slots = []
    for s, sl in enumerate(seq_lens):
        pos = np.arange(int(sl), dtype=np.int64)
        slots.append(bt[s, pos // block_size].astype(np.int64) * block_size + pos % block_size)
    slots = np.concatenate(slots) if slots else np.zeros(0, np.int64)
    if host_values:
        k = rng.standard_normal((ntok, Hkv, D), dtype=np.float32)
        v = rng.standard_normal((ntok, Hkv, D), dtype=np.float32)
        q = rng.standard_normal((T, Hq, D), dtype=np.float32)
        b.key = torch.from_numpy(k).to(td).to(dev)
        b.value = torch.from_numpy(v).to(td).to(dev)
        b.query = torch.from_numpy(q).to(td).to(dev)
    else:
        g = torch.Generator(device=dev)
        g.manual_seed(seed)
        b.key = torch.randn((ntok, Hkv, D), generator=g, device=dev, dtype=torch.float32).to(td)
        b.value = torch.randn((ntok, Hkv, D), generator=g, device=dev, dtype=torch.float32).to(td)
        b.query = torch.randn((T, Hq, D), generator=g, device=dev, dtype=torch.float32).to(td)
    b.slot_mapping = torch.from_numpy(slots).to(dev)
    b.kv_cache = gfx906_fa.new_kv_cache(nb, block_size, Hkv, D, device=dev)
    b.block_table = torch.from_numpy(bt).to(dev)
    b.seq_lens_t = torch.from_numpy(seq_lens).to(dev)
    b.qsl_t = torch.from_numpy(b.qsl).to(dev)
    if write_cache:
        kp, vp = b.planes()
        gfx906_fa.reshape_and_cache_q8_kv(b.key, b.value, b.slot_mapping, kp, vp)
    return b


def attention(b: Batch, out: Optional[torch.Tensor] = None, workspace=None,
              out_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    kp, vp = b.planes()
    return gfx906_fa.paged_attention(b.query, kp, vp, b.block_table, b.seq_lens_t, b.qsl_t,
                                     b.max_query_len, b.max_seq_len, b.scale, out=out,
                                     workspace=workspace, out_dtype=out_dtype)


def sub_batch(b: Batch, s0: int, s1: int) -> Batch:
    """The sequences [s0, s1) of a batch as a batch of their own over the same
    KV cache (their query tokens are contiguous in the varlen layout)."""
    qsl = b.qsl
    t0, t1 = int(qsl[s0]), int(qsl[s1])
    sb = Batch(Hq=b.Hq, Hkv=b.Hkv, D=b.D, block_size=b.block_size, seq_lens=b.seq_lens[s0:s1].copy(),
               q_lens=b.q_lens[s0:s1].copy(), block_table_np=b.block_table_np[s0:s1].copy(),
               num_blocks=b.num_blocks, dtype=b.dtype, scale=b.scale, device=b.device)
    sb.query = b.query[t0:t1]
    sb.kv_cache = b.kv_cache
    sb.block_table = b.block_table[s0:s1].contiguous()
    sb.seq_lens_t = b.seq_lens_t[s0:s1].contiguous()
    sb.qsl_t = torch.from_numpy(sb.qsl).to(b.device)
    return sb


def rope_cos_sin_cache(max_position: int, rot_dim: int, dtype: torch.dtype, device,
                       base: float = 10000.0) -> torch.Tensor:
    """[max_position, rot_dim] table cos | sin of position * base^(-2i/rot_dim),
    the layout of vLLM's rotary cos_sin_cache (synthetic bench input)."""
    inv = 1.0 / (base ** (torch.arange(0, rot_dim, 2, dtype=torch.float32) / rot_dim))
    f = torch.outer(torch.arange(max_position, dtype=torch.float32), inv)
    return torch.cat([f.cos(), f.sin()], dim=-1).to(dtype).to(device)


def rope_write_bytes(T: int, Hq: int, Hkv: int, D: int = 128, rot: int = 128, elem: int = 2) -> int:
    """Algorithmic HBM bytes of the fused rotary + K/V cache write over T
    tokens: query and key read and written back, value read, the Q8_0 K and
    V rows written (2 x 136 B per kv-head), one cos/sin row, position and slot."""
    return T * ((Hq + Hkv) * D * elem * 2 + Hkv * D * elem + Hkv * 2 * (D // 32 * 34) + rot * elem + 16)


# ---------------------------------------------------------------------------
# The benchmark configurations
# ---------------------------------------------------------------------------
CONFIGS = {
    "cfg1": "1 seq x 1024 tokens, 8/1 heads, fp16, single-token decode",
    "cfg2": "32 seqs, ctx U[2048,16384], 48/8 heads, fp16 Q, Q8 K/V, decode",
    "cfg3": "1 seq x 32768 causal prefill, 48/8 heads, bf16",
    "cfg4": "4 chunks x 2048 (prior 0/16K/32K/64K) + 60 decodes ctx logU[1K,128K], 48/8, fp16",
    "cfg5": "8 seqs x 131072 cached + 5 verify tokens, 6/1 heads (and 48/8), fp16",
    "cfg5k6": "8 seqs x 131072 cached + 6 verify tokens (n-gram k=5), 6/1 heads, fp16",
}


def cfg_shape(name: str, seed: int = 0, heads=None):
    """-> (seq_lens, q_lens, Hq, Hkv, dtype) for a configuration."""
    rng = np.random.default_rng(1000 + seed)
    if name == "cfg1":
        return [1024], [1], 8, 1, "f16"
    if name == "cfg2":
        sl = rng.integers(2048, 16384 + 1, size=32)
        return sl.tolist(), [1] * 32, 48, 8, "f16"
    if name == "cfg3":
        return [32768], [32768], 48, 8, "bf16"
    if name == "cfg4":
        prior = [0, 16384, 32768, 65536]
        sl = [p + 2048 for p in prior]
        ql = [2048] * 4
        dec = np.exp(rng.uniform(math.log(1024), math.log(131072), size=60)).astype(np.int64)
        return sl + dec.tolist(), ql + [1] * 60, 48, 8, "f16"
    if name in ("cfg5", "cfg5k6"):
        # cfg5k6: the verify step of the reference's n-gram serving setting,
        # num_speculative_tokens = 5 plus the bonus token (36 rows at 6/1)
        hq, hkv = heads or (6, 1)
        nq = 5 if name == "cfg5" else 6
        return [131072 + nq] * 8, [nq] * 8, hq, hkv, "f16"
    raise KeyError(name)


def build_cfg(name: str, device="cuda", seed: int = 0, heads=None, host_values=None) -> Batch:
    sl, ql, hq, hkv, dt = cfg_shape(name, seed, heads)
    if host_values is None:
        host_values = sum(sl) * hkv <= 1 << 16
    return build_batch(sl, ql, hq, hkv, dtype=dt, seed=seed, device=device, host_values=host_values)
