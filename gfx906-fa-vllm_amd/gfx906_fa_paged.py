"""Host dispatcher for the Q8_0 paged-attention backend (MI355X).

Mirror of ``extension/gfx906_fa_paged.py`` (``forward_paged``, lines 197-465).
The reference pads Q per sequence with a host sync each (lines 264-286),
chooses between direct-paged / fused-gather / legacy paths (lines 56-70,
255-376) and unpads the fp32 result (lines 322-330).  Here every batch -
decode, chunked prefill, mixed, speculative verify - is one varlen call
into the HIP library: the kernels read ``query_start_loc`` and ``seq_lens``
on the device, write ``[T, Hq, D]`` directly in the output dtype, and apply
the reference's causal rule (row j of sequence s sees keys
k <= seq_lens[s] - n_q[s] + j, lines 288-295) inline.

Also holds the mapping between vLLM's per-layer KV tensor and the planar Q8
planes (``q8_planes``).
"""
from __future__ import annotations

import math
import os
import time
from typing import Optional, Tuple

import torch

import gfx906_fa

SUBPAGE_TOKENS = gfx906_fa.SUBPAGE_TOKENS
SUBPAGE_BYTES = gfx906_fa.SUBPAGE_BYTES

# GFX906_FA_FWD_DEBUG=1: one line per forward_paged call (shapes before the
# launch, then OK or FAILED with the error) appended to
# /tmp/gfx906_fa_debug/fwd-<pid>.log, with the device synchronized around the
# launch so an asynchronous fault is reported by the call that caused it
# (extension/gfx906_fa_paged.py:23,72-80,297-320).
_DBG = os.environ.get("GFX906_FA_FWD_DEBUG", "0") == "1"
_DBG_DIR = "/tmp/gfx906_fa_debug"


def _fwdlog(msg: str) -> None:
    if not _DBG:
        return
    try:
        os.makedirs(_DBG_DIR, exist_ok=True)
        with open(os.path.join(_DBG_DIR, f"fwd-{os.getpid()}.log"), "a") as f:
            f.write(f"[{time.time():.3f}] {msg}\n")
    except OSError:
        pass


def plane_bytes_per_head(block_size: int) -> int:
    """Bytes of one (page, kv-head) in one plane: block_size/16 sub-pages."""
    return block_size // SUBPAGE_TOKENS * SUBPAGE_BYTES


def q8_planes(kv_cache: torch.Tensor, num_kv_heads: int, head_size: int,
              block_size: Optional[int] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """(K plane, V plane) uint8 views [NB, Hkv, block_size/16*2176] of a KV tensor.

    Accepted layouts:
      * the planar cache itself, uint8 [NB, 2, Hkv, block_size/16*2176]
        (``gfx906_fa.new_kv_cache``);
      * the backend's "q8_0" page, uint8 [NB, 2, Hkv, block_size/16, 2176]
        (``Gfx906FABackend.get_kv_cache_shape(..., "q8_0")``): the same bytes
        as the planar cache, viewed with the sub-page as its own dimension;
      * vLLM's per-layer tensor [NB, 2, bs, Hkv, D] in fp16/bf16/fp32
        (``Gfx906FABackend.get_kv_cache_shape``, identical to the reference's
        ``extension/gfx906_fa_backend.py:153-165``).  Each page's bytes hold
        the K plane then the V plane of that page; 136/256 of an fp16 page is
        used (the "q8_0" page above holds the same bytes with no slack).
    """
    if kv_cache.dtype == torch.uint8 and kv_cache.dim() == 5:
        NB, two, Hkv, nsp, sub = kv_cache.shape
        if two != 2 or Hkv != num_kv_heads or sub != SUBPAGE_BYTES or head_size != 128:
            raise RuntimeError("q8_0 pages must be uint8 [NB, 2, Hkv, bs/16, 2176] (head_size 128)")
        if block_size is not None and nsp * SUBPAGE_TOKENS != block_size:
            raise RuntimeError(f"block_size mismatch {nsp * SUBPAGE_TOKENS} vs {block_size}")
        if kv_cache.stride(4) != 1 or kv_cache.stride(3) != SUBPAGE_BYTES:
            raise RuntimeError("q8_0 pages must be contiguous within a kv-head")
        kv_cache = kv_cache.flatten(3)
    if kv_cache.dtype == torch.uint8 and kv_cache.dim() == 4:
        if kv_cache.shape[1] != 2 or kv_cache.shape[2] != num_kv_heads:
            raise RuntimeError("planar cache must be [NB, 2, Hkv, bs/16*2176]")
        return kv_cache[:, 0], kv_cache[:, 1]
    if kv_cache.dim() != 5 or kv_cache.shape[1] != 2:
        raise RuntimeError("kv_cache must be [num_blocks, 2, block_size, Hkv, D]")
    if not kv_cache.is_contiguous():
        raise RuntimeError("kv_cache must be contiguous")
    NB, _, bs, Hkv, D = kv_cache.shape
    if block_size is not None and bs != block_size:
        raise RuntimeError(f"block_size mismatch {bs} vs {block_size}")
    if Hkv != num_kv_heads or D != head_size or head_size != 128:
        raise RuntimeError("kv_cache head shape mismatch (head_size must be 128)")
    if bs % SUBPAGE_TOKENS != 0:
        raise RuntimeError("block_size must be a multiple of 16")
    page = kv_cache.view(torch.uint8).view(NB, -1)
    pb = plane_bytes_per_head(bs)
    if 2 * Hkv * pb > page.shape[1]:
        raise RuntimeError("kv_cache page too small for the Q8 planes")
    k = page[:, : Hkv * pb].view(NB, Hkv, pb)            # views keep the page stride
    v = page[:, Hkv * pb: 2 * Hkv * pb].view(NB, Hkv, pb)
    return k, v


def forward_paged(
    query: torch.Tensor,                 # [num_tokens, Hq, D]   fp16 / bf16 / fp32
    key_cache: torch.Tensor,             # K plane [NB, Hkv, bs/16*2176] uint8
    value_cache: torch.Tensor,           # V plane [NB, Hkv, bs/16*2176] uint8
    block_table: torch.Tensor,           # [num_seqs, max_blocks]  int32
    seq_lens: torch.Tensor,              # [num_seqs]              int32
    cu_seqlens_q: torch.Tensor,          # [num_seqs+1]            int32
    max_seqlen_q: int,
    max_seqlen_k: int,
    scale: Optional[float] = None,
    key_cache_q8: Optional[torch.Tensor] = None,
    q_pad_buf: Optional[torch.Tensor] = None,
    mask_buf: Optional[torch.Tensor] = None,
    k_gather_buf: Optional[torch.Tensor] = None,
    v_gather_buf: Optional[torch.Tensor] = None,
    *,
    out: Optional[torch.Tensor] = None,
    workspace: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """vLLM-shaped paged attention; returns ``[num_tokens, Hq*D]``.

    ``out`` (``[num_tokens, Hq, D]`` or ``[num_tokens, Hq*D]``, any of
    fp32/fp16/bf16) is written in place when given; otherwise an fp32 tensor
    is returned like the reference's.  ``key_cache_q8``, ``q_pad_buf``,
    ``mask_buf``, ``k_gather_buf`` and ``v_gather_buf`` are accepted for call
    compatibility with the reference and unused: nothing is padded or
    gathered.  ``key_cache_q8``, if given, must be ``key_cache``."""
    if key_cache_q8 is not None and key_cache_q8.data_ptr() != key_cache.data_ptr():
        raise RuntimeError("key_cache_q8 must alias key_cache (K is always Q8_0 here)")
    num_tokens, Hq, D = query.shape
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    bt = block_table if block_table.dtype == torch.int32 else block_table.to(torch.int32)
    sl = seq_lens if seq_lens.dtype == torch.int32 else seq_lens.to(torch.int32)
    cu = cu_seqlens_q if cu_seqlens_q.dtype == torch.int32 else cu_seqlens_q.to(torch.int32)
    if bt.stride(-1) != 1:
        bt = bt.contiguous()
    o3 = None
    if out is not None:
        o3 = out.view(out.shape[0], Hq, D)
    if _DBG:
        _fwdlog(f"forward_paged VARLEN: num_tokens={num_tokens} Hq={Hq} Hkv={key_cache.shape[1]} D={D} "
                f"num_seqs={sl.shape[0]} Sq_max={max_seqlen_q} Sk_max={max_seqlen_k} "
                f"q_dtype={query.dtype} out={None if out is None else (tuple(out.shape), out.dtype)} "
                f"scale={scale}")
        if query.is_cuda:
            torch.cuda.synchronize(query.device)
    try:
        res = gfx906_fa.paged_attention(query, key_cache, value_cache, bt, sl.contiguous(), cu.contiguous(),
                                        max_seqlen_q, max_seqlen_k, scale, out=o3, workspace=workspace,
                                        out_dtype=torch.float32)
        if _DBG:
            if query.is_cuda:
                torch.cuda.synchronize(query.device)
            _fwdlog(f"forward_paged OK: out={tuple(res.shape)}")
    except Exception as e:
        _fwdlog(f"forward_paged FAILED: {e!r}")
        raise
    return res.view(res.shape[0], Hq * D)
