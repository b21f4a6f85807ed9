"""``gfx906_fa`` op module for MI355X (gfx950).

Mirrors the reference's pybind11 module (``extension/gfx906_fa.cpp:660-690``):
same op names, argument names, defaults and error behaviour (a failed check
raises ``RuntimeError``, as ``TORCH_CHECK`` does).  Each op validates its
tensors, then calls one ``extern "C"`` entry point of ``libgfx906_fa_amd.so``
(declared in ``include/gfx906_fa_amd.h``) on the current HIP stream.  There
is no CPU fallback: importing this module without the built library, or
calling an op on a CPU tensor, raises.

Ops
---
quantize_q8_0(k_fp16)                                  extension/gfx906_fa.cpp:273-309
reshape_and_cache_q8(key, slot_mapping, k_cache_q8)    extension/gfx906_fa.cpp:322-374
gather_paged_kv_q8(key_cache_q8, value_cache, block_table, seq_lens, Sk,
                   k_out=None, v_out=None)             extension/gfx906_fa.cpp:393-498
forward(q, k_q8, v_fp16, scale, kv_max=None, mask=None, q_abs_offset=None)
                                                       extension/gfx906_fa.cpp:120-265
forward_paged_direct(q, key_cache_q8, value_cache, block_table, seq_lens,
                     scale, mask=None, q_abs_offset=None)
                                                       extension/gfx906_fa.cpp:516-658
New for the Q8 K+V cache of this backend:
reshape_and_cache_q8_kv(key, value, slot_mapping, key_cache, value_cache)
rope_and_cache_q8_kv(positions, query, key, value, cos_sin_cache, is_neox,
                     slot_mapping, key_cache, value_cache, rot_dim=None)
gather_paged_kv_q8q8(key_cache, value_cache, block_table, seq_lens, Sk, ...)
paged_attention(query, key_cache, value_cache, block_table, seq_lens,
                query_start_loc, max_query_len, max_seq_len, scale, out=None, ...)
new_kv_cache(num_blocks, block_size, num_kv_heads, head_size=128, device=...)
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("GFX906_FA_AMD_LIB") or os.path.join(_HERE, "libgfx906_fa_amd.so")

QK8_0 = 32
Q8_0_BYTES = 34
SUBPAGE_TOKENS = 16
SUBPAGE_BYTES = 2176

_DT = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}

_lib = None


def _load():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"gfx906_fa: HIP library not built ({LIB_PATH}); run "
            "`python gfx906-fa-vllm_amd/build.py` (or __graft_entry__.build())")
    L = ctypes.CDLL(LIB_PATH)
    P, I, I64, F, SZ = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_float, ctypes.c_size_t
    sig = {
        "gfx906_fa_amd_version": (ctypes.c_char_p, []),
        "launch_quantize_q8_0_dense": (I, [P, P, I, I, P]),
        "gfx906_fa_amd_quantize_q8_0": (I, [P, I, P, I64, I, P]),
        "launch_reshape_and_cache_q8": (I, [P, P, P, I, I, I, I, I64, I64, I64, I64, I64, P]),
        "gfx906_fa_amd_reshape_and_cache_q8": (I, [P, I, P, P, I, I, I, I, I64, I64, I64, I64, I64, P]),
        "launch_gather_paged_kv_q8": (I, [P, P, P, P, P, P, I, I, I, I, I, I, I,
                                          I64, I64, I64, I64, I64, I64, P]),
        "gfx906_fa_amd_gather_rows": (I, [P, P, P, P, P, P, I, I, I, I, I, I, I,
                                          I64, I64, I64, I64, I64, I64, P]),
        "gfx906_fa_amd_gather_planar": (I, [P, P, P, P, P, P, I, I, I, I, I, I, I64, I64, P]),
        "gfx906_fa_amd_cache_write_kv": (I, [P, P, I, P, P, P, I, I, I, I,
                                             I64, I64, I64, I64, I64, I64, P]),
        "gfx906_fa_amd_rope_cache_write_kv": (I, [P, P, P, I, P, P, I, I64, I, I, I, P, P, P, I, I, I, I, I,
                                                  I64, I64, I64, I64, I64, I64, I64, I64, P]),
        "gfx906_fa_amd_paged_attention_workspace_size": (SZ, [I, I, I, I, I, I, I]),
        "gfx906_fa_amd_paged_attention_workspace_bound": (SZ, [I, I64, I, I, I]),
        "gfx906_fa_amd_paged_attention_plan_info": (I, [I, I, I, I, I, I, I, P, I]),
        "gfx906_fa_amd_paged_attention_workspace_bound_info": (I, [I, I64, I, I, I, I64, P, I]),
        "gfx906_fa_amd_device_cus": (I, []),
        "gfx906_fa_amd_stream_read_words": (I, []),
        "gfx906_fa_amd_stream_read": (I, [P, I64, P, I, P]),
        "gfx906_fa_amd_noalloc_scratch_copy": (I, [P, SZ, SZ, P]),
        "gfx906_fa_amd_paged_attention_noalloc": (I, [P, I, I64, I64, P, P, I64, I64, P, I64, P, P, P,
                                                      I, I, I, I, I, I, I, I, I, F, P, I, I64, I64, P]),
        "gfx906_fa_amd_paged_attention": (I, [P, I, I64, I64, P, P, I64, I64, P, I64, P, P, P,
                                              I, I, I, I, I, I, I, I, I, F, P, I, I64, I64, P, SZ, P]),
        "gfx906_fa_amd_paged_attention_kv_write": (I, [P, I, I64, I64, P, P, I64, I64, P, I64, P, P, P,
                                                       I, I, I, I, I, I, I, I, I, F, P, I, I64, I64, P, SZ,
                                                       P, P, I, I64, I64, I64, I64, P, P]),
        "gfx906_fa_amd_pack_flat_kv": (I, [P, P, P, P, I, I, I, P]),
        "gfx906_fa_amd_flat_decode_workspace_size": (SZ, [I, I, I, I, I]),
        "gfx906_fa_amd_flat_decode": (I, [P, I, I64, I64, P, P, P, P, I, I, I, I, I, I, F, P, I64, I64,
                                          P, SZ, P]),
        "gfx906_fa_amd_paged_attention_tiled": (I, [P, I, I64, I64, P, P, I, I64, I64, I64, I64, P, I64,
                                                    P, P, P, I, P, I64, I64, I, I, I, I, I, I, I, I,
                                                    F, P, I64, I64, P]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


def lib():
    return _load()


def library_path() -> str:
    return LIB_PATH


def _check(cond: bool, msg: str) -> None:
    if not cond:
        raise RuntimeError(msg)


def _cuda(t: torch.Tensor, name: str) -> None:
    _check(t.is_cuda, f"{name} must be CUDA/HIP")


def _ptr(t: Optional[torch.Tensor]):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(dev: torch.device):
    return ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)


def _ok(err: int, what: str) -> None:
    if err != 0:
        raise RuntimeError(f"{what} failed: hipError {err}")


# ---------------------------------------------------------------------------
# Reference ops
# ---------------------------------------------------------------------------
def quantize_q8_0(k_fp16: torch.Tensor) -> torch.Tensor:
    """Dense Q8_0 quantize of the last dim (fp16; bf16 / fp32 also accepted).
    ``extension/gfx906_fa.cpp:273-309``."""
    _cuda(k_fp16, "k_fp16")
    _check(k_fp16.is_contiguous(), "k_fp16 must be contiguous")
    _check(k_fp16.dtype in _DT, "k_fp16 must be fp16 (or bf16 / fp32)")
    _check(k_fp16.dim() >= 1, "k_fp16 must have at least 1 dim")
    D = k_fp16.shape[-1]
    _check(D % QK8_0 == 0, "last dim must be multiple of 32")
    N = k_fp16.numel() // D if D else 0
    out = torch.empty((*k_fp16.shape[:-1], D // QK8_0 * Q8_0_BYTES), dtype=torch.uint8,
                      device=k_fp16.device)
    err = _load().gfx906_fa_amd_quantize_q8_0(_ptr(k_fp16), _DT[k_fp16.dtype], _ptr(out), N, D,
                                              _stream(k_fp16.device))
    _ok(err, "gfx906_fa_amd_quantize_q8_0")
    return out


def reshape_and_cache_q8(key: torch.Tensor, slot_mapping: torch.Tensor,
                         k_cache_q8: torch.Tensor) -> None:
    """Quantize key [T, Hkv, D] and scatter AoS rows into
    k_cache_q8 [NB, bs, Hkv, (D/32)*34] at slot_mapping (int64, < 0 skips).
    Strides of both tensors are honoured.  ``extension/gfx906_fa.cpp:322-374``."""
    for t, n in ((key, "key"), (slot_mapping, "slot_mapping"), (k_cache_q8, "k_cache_q8")):
        _cuda(t, n)
    _check(key.dtype in _DT, "key must be fp16 (or bf16 / fp32)")
    _check(slot_mapping.dtype == torch.int64, "slot_mapping must be int64")
    _check(k_cache_q8.dtype == torch.uint8, "k_cache_q8 must be uint8")
    _check(key.dim() == 3, "key must be [num_tokens, Hkv, D]")
    _check(k_cache_q8.dim() == 4, "k_cache_q8 must be [B, bs, Hkv, bytes]")
    T, Hkv, D = key.shape
    _check(D % QK8_0 == 0, "head_size must be multiple of 32")
    bpr = D // QK8_0 * Q8_0_BYTES
    _check(k_cache_q8.shape[2] == Hkv,
           f"k_cache_q8 Hkv mismatch: got {k_cache_q8.shape[2]} vs key Hkv={Hkv}")
    _check(k_cache_q8.shape[3] == bpr,
           f"k_cache_q8 last dim mismatch: got {k_cache_q8.shape[3]} expected {bpr}")
    _check(k_cache_q8.stride(3) == 1, "k_cache_q8 rows must be contiguous")
    _check(key.stride(2) == 1, "key rows must be contiguous")
    _check(slot_mapping.shape[0] == T, "slot_mapping length mismatch")
    sm = slot_mapping.contiguous()
    err = _load().gfx906_fa_amd_reshape_and_cache_q8(
        _ptr(key), _DT[key.dtype], _ptr(sm), _ptr(k_cache_q8), T, Hkv, D, k_cache_q8.shape[1],
        key.stride(0), key.stride(1), k_cache_q8.stride(0), k_cache_q8.stride(1),
        k_cache_q8.stride(2), _stream(key.device))
    _ok(err, "launch_reshape_and_cache_q8")


def gather_paged_kv_q8(key_cache_q8: torch.Tensor, value_cache: torch.Tensor,
                       block_table: torch.Tensor, seq_lens: torch.Tensor, Sk: int,
                       k_out: Optional[torch.Tensor] = None,
                       v_out: Optional[torch.Tensor] = None):
    """Paged AoS K (Q8_0 rows) + paged V rows -> contiguous BHSD
    [k_out, v_out].  V rows past seq_lens (or on a -1 page) are zeroed, K rows
    there are left as they were.  value_cache may be fp16 [NB, bs, Hkv, D]
    (the reference contract) or uint8 AoS Q8_0 rows [NB, bs, Hkv, (D/32)*34]
    (the Q8/Q8 variant).  Caller buffers are used only on an exact
    shape/dtype/contiguity match (``extension/gfx906_fa.cpp:449-469``).
    ``extension/gfx906_fa.cpp:393-498``."""
    for t, n in ((key_cache_q8, "key_cache_q8"), (value_cache, "value_cache"),
                 (block_table, "block_table"), (seq_lens, "seq_lens")):
        _cuda(t, n)
    _check(key_cache_q8.dtype == torch.uint8, "key_cache_q8 must be uint8")
    _check(value_cache.dtype in (torch.float16, torch.uint8), "value_cache must be fp16 (or uint8 Q8_0 rows)")
    _check(seq_lens.dtype == torch.int32, "seq_lens must be int32")
    _check(key_cache_q8.dim() == 4, "key_cache_q8 must be 4D")
    _check(value_cache.dim() == 4, "value_cache must be 4D")
    NB, bs, Hkv, bpr = key_cache_q8.shape
    vq8 = value_cache.dtype == torch.uint8
    D = (value_cache.shape[3] // Q8_0_BYTES * QK8_0) if vq8 else value_cache.shape[3]
    _check(value_cache.shape[0] == NB, "value_cache blocks mismatch")
    _check(value_cache.shape[1] == bs, "value_cache block_size mismatch")
    _check(value_cache.shape[2] == Hkv, "value_cache Hkv mismatch")
    _check(D % QK8_0 == 0, "D must be multiple of 32")
    _check(bpr == D // QK8_0 * Q8_0_BYTES,
           f"bytes_per_row must equal (D/32)*34, got {bpr} vs expected {D // QK8_0 * Q8_0_BYTES}")
    _check(block_table.dtype == torch.int32, "block_table must be int32 (caller should .to(torch.int32))")
    _check(block_table.is_contiguous(), "block_table must be contiguous")
    _check(seq_lens.is_contiguous(), "seq_lens must be contiguous")
    B, M = block_table.shape
    _check(seq_lens.shape[0] == B, "seq_lens vs block_table batch mismatch")
    _check(Sk > 0 and Sk % 32 == 0, f"Sk must be positive multiple of 32, got {Sk}")
    _check(key_cache_q8.stride(3) == 1 and value_cache.stride(3) == 1, "cache rows must be contiguous")
    vrow = value_cache.shape[3]

    def use_or_alloc(buf, dtype, dim3):
        if (buf is not None and buf.dim() == 4 and tuple(buf.shape) == (B, Hkv, Sk, dim3)
                and buf.dtype == dtype and buf.device == key_cache_q8.device and buf.is_contiguous()):
            return buf
        return torch.empty((B, Hkv, Sk, dim3), dtype=dtype, device=key_cache_q8.device)

    k_o = use_or_alloc(k_out, torch.uint8, bpr)
    v_o = use_or_alloc(v_out, value_cache.dtype, vrow)
    es = value_cache.element_size()
    err = _load().gfx906_fa_amd_gather_rows(
        _ptr(key_cache_q8), _ptr(value_cache), _ptr(block_table), _ptr(seq_lens), _ptr(k_o),
        _ptr(v_o), B, Hkv, Sk, bpr, vrow * es, bs, M,
        key_cache_q8.stride(0), key_cache_q8.stride(1), key_cache_q8.stride(2),
        value_cache.stride(0) * es, value_cache.stride(1) * es, value_cache.stride(2) * es,
        _stream(key_cache_q8.device))
    _ok(err, "launch_gather_paged_kv_q8")
    return [k_o, v_o]


# ---------------------------------------------------------------------------
# Planar Q8 K+V cache of this backend
# ---------------------------------------------------------------------------
def new_kv_cache(num_blocks: int, block_size: int, num_kv_heads: int, head_size: int = 128,
                 device=None) -> torch.Tensor:
    """Zeroed planar cache uint8 [NB, 2, Hkv, block_size/16*2176]
    (dim 1: 0 = K plane, 1 = V plane)."""
    _check(head_size == 128, "the planar Q8 cache supports head_size 128")
    _check(block_size % SUBPAGE_TOKENS == 0, "block_size must be a multiple of 16")
    return torch.zeros((num_blocks, 2, num_kv_heads, block_size // SUBPAGE_TOKENS * SUBPAGE_BYTES),
                       dtype=torch.uint8, device=device)


def _plane_info(key_cache: torch.Tensor, value_cache: torch.Tensor):
    """Validates a planar (K, V) plane pair [NB, Hkv, bs/16*2176] (uint8, any
    block/head strides, contiguous pages) -> (block_size, Hkv, block stride,
    head stride)."""
    _check(key_cache.dtype == torch.uint8 and value_cache.dtype == torch.uint8,
           "key_cache / value_cache must be uint8 planar Q8 planes")
    _check(key_cache.dim() == 3 and value_cache.dim() == 3,
           "key_cache / value_cache must be [num_blocks, Hkv, block_size/16*2176]")
    _check(key_cache.shape == value_cache.shape, "key_cache / value_cache shape mismatch")
    _check(key_cache.stride() == value_cache.stride(), "key_cache / value_cache stride mismatch")
    NB, Hkv, nbytes = key_cache.shape
    _check(nbytes % SUBPAGE_BYTES == 0, "page bytes must be a multiple of 2176")
    _check(key_cache.stride(2) == 1, "pages must be contiguous")
    return nbytes // SUBPAGE_BYTES * SUBPAGE_TOKENS, Hkv, key_cache.stride(0), key_cache.stride(1)


def reshape_and_cache_q8_kv(key: torch.Tensor, value: torch.Tensor, slot_mapping: torch.Tensor,
                            key_cache: torch.Tensor, value_cache: torch.Tensor) -> None:
    """Quantize key and value [T, Hkv, 128] to Q8_0 and write them at
    slot_mapping into the planar planes (one launch; slot < 0 skips)."""
    for t, n in ((key, "key"), (value, "value"), (slot_mapping, "slot_mapping"),
                 (key_cache, "key_cache"), (value_cache, "value_cache")):
        _cuda(t, n)
    _check(key.dtype in _DT and value.dtype == key.dtype, "key/value must share dtype fp16/bf16/fp32")
    _check(key.dim() == 3 and value.shape == key.shape, "key/value must be [num_tokens, Hkv, D]")
    _check(slot_mapping.dtype == torch.int64, "slot_mapping must be int64")
    T, Hkv, D = key.shape
    _check(D == 128, "head_size must be 128")
    _check(key.stride(2) == 1 and value.stride(2) == 1, "key/value rows must be contiguous")
    _check(slot_mapping.shape[0] == T, "slot_mapping length mismatch")
    bs, Hc, cbs, chs = _plane_info(key_cache, value_cache)
    _check(Hc == Hkv, f"cache Hkv mismatch: got {Hc} vs key Hkv={Hkv}")
    sm = slot_mapping.contiguous()
    err = _load().gfx906_fa_amd_cache_write_kv(
        _ptr(key), _ptr(value), _DT[key.dtype], _ptr(sm), _ptr(key_cache), _ptr(value_cache), T,
        Hkv, D, bs, key.stride(0), key.stride(1), value.stride(0), value.stride(1), cbs, chs,
        _stream(key.device))
    _ok(err, "gfx906_fa_amd_cache_write_kv")


def rope_and_cache_q8_kv(positions: torch.Tensor, query: torch.Tensor, key: torch.Tensor,
                         value: torch.Tensor, cos_sin_cache: torch.Tensor, is_neox: bool,
                         slot_mapping: torch.Tensor, key_cache: torch.Tensor,
                         value_cache: torch.Tensor, rot_dim: Optional[int] = None) -> None:
    """Rotary embedding of query [T, Hq, 128] and key [T, Hkv, 128] in place
    (vLLM semantics: cos/sin rows of cos_sin_cache [max_position, rot_dim]
    at ``positions`` (int64), converted to the model dtype; neox or GPT-J
    pairs; per-operation rounding in the model dtype), then the rotated key
    and the value quantized to Q8_0 at slot_mapping (< 0 skips) - one launch.
    Positions outside [0, max_position) leave their rows unrotated."""
    for t, n in ((positions, "positions"), (query, "query"), (key, "key"), (value, "value"),
                 (cos_sin_cache, "cos_sin_cache"), (slot_mapping, "slot_mapping"),
                 (key_cache, "key_cache"), (value_cache, "value_cache")):
        _cuda(t, n)
    _check(query.dtype in (torch.float16, torch.bfloat16) and key.dtype == query.dtype
           and value.dtype == query.dtype, "query/key/value must share dtype fp16 or bf16")
    _check(query.dim() == 3 and key.dim() == 3 and value.shape == key.shape and query.shape[0] == key.shape[0],
           "query must be [T, Hq, D], key/value [T, Hkv, D]")
    _check(positions.dtype == torch.int64 and positions.dim() == 1 and positions.shape[0] == query.shape[0],
           "positions must be int64 [num_tokens]")
    _check(slot_mapping.dtype == torch.int64 and slot_mapping.shape[0] == query.shape[0],
           "slot_mapping must be int64 [num_tokens]")
    _check(cos_sin_cache.dtype in _DT and cos_sin_cache.dim() == 2 and cos_sin_cache.stride(1) == 1,
           "cos_sin_cache must be [max_position, rot_dim] with contiguous rows")
    T, Hq, D = query.shape
    Hkv = key.shape[1]
    _check(D == 128 and key.shape[2] == 128, "head_size must be 128")
    for t, n in ((query, "query"), (key, "key"), (value, "value")):
        _check(t.stride(2) == 1, f"{n} rows must be contiguous")
    rot = cos_sin_cache.shape[1] if rot_dim is None else int(rot_dim)
    bs, Hc, cbs, chs = _plane_info(key_cache, value_cache)
    _check(Hc == Hkv, f"cache Hkv mismatch: got {Hc} vs key Hkv={Hkv}")
    _check(Hq % Hkv == 0, f"heads_q={Hq} must be divisible by heads_kv={Hkv}")
    pos = positions.contiguous()
    sm = slot_mapping.contiguous()
    err = _load().gfx906_fa_amd_rope_cache_write_kv(
        _ptr(query), _ptr(key), _ptr(value), _DT[query.dtype], _ptr(pos), _ptr(cos_sin_cache),
        _DT[cos_sin_cache.dtype], cos_sin_cache.stride(0), cos_sin_cache.shape[0], rot, 1 if is_neox else 0,
        _ptr(sm), _ptr(key_cache), _ptr(value_cache), T, Hq, Hkv, D, bs,
        query.stride(0), query.stride(1), key.stride(0), key.stride(1), value.stride(0), value.stride(1),
        cbs, chs, _stream(query.device))
    _ok(err, "gfx906_fa_amd_rope_cache_write_kv")


def gather_paged_kv_q8q8(key_cache: torch.Tensor, value_cache: torch.Tensor,
                         block_table: torch.Tensor, seq_lens: torch.Tensor, Sk: int,
                         k_out: Optional[torch.Tensor] = None,
                         v_out: Optional[torch.Tensor] = None):
    """Planar Q8 K+V planes -> contiguous AoS Q8_0 rows [B, Hkv, Sk, 136] for K
    and V, with the validity rule of ``gather_paged_kv_q8`` (V zeroed, K kept
    on invalid tokens)."""
    for t, n in ((key_cache, "key_cache"), (value_cache, "value_cache"),
                 (block_table, "block_table"), (seq_lens, "seq_lens")):
        _cuda(t, n)
    _check(block_table.dtype == torch.int32 and block_table.is_contiguous(),
           "block_table must be contiguous int32")
    _check(seq_lens.dtype == torch.int32 and seq_lens.is_contiguous(), "seq_lens must be contiguous int32")
    bs, Hkv, cbs, chs = _plane_info(key_cache, value_cache)
    B, M = block_table.shape
    _check(seq_lens.shape[0] == B, "seq_lens vs block_table batch mismatch")
    _check(Sk > 0 and Sk % 32 == 0, f"Sk must be positive multiple of 32, got {Sk}")

    def use_or_alloc(buf):
        if (buf is not None and tuple(buf.shape) == (B, Hkv, Sk, 136) and buf.dtype == torch.uint8
                and buf.device == key_cache.device and buf.is_contiguous()):
            return buf
        return torch.empty((B, Hkv, Sk, 136), dtype=torch.uint8, device=key_cache.device)

    k_o, v_o = use_or_alloc(k_out), use_or_alloc(v_out)
    err = _load().gfx906_fa_amd_gather_planar(
        _ptr(key_cache), _ptr(value_cache), _ptr(block_table), _ptr(seq_lens), _ptr(k_o),
        _ptr(v_o), B, Hkv, Sk, 128, bs, M, cbs, chs, _stream(key_cache.device))
    _ok(err, "gfx906_fa_amd_gather_planar")
    return [k_o, v_o]


def new_workspace(nbytes: int, device) -> torch.Tensor:
    """Attention workspace (decode plan + partial results of split
    segments; each call writes what it reads, so no initial contents are
    needed).  Reuse it across calls on one stream; calls that overlap on
    different streams need their own."""
    return torch.empty(max(int(nbytes), 256), dtype=torch.uint8, device=device)


def workspace_size(num_seqs: int, num_tokens: int, num_heads: int, num_kv_heads: int,
                   max_query_len: int, max_seq_len: int, head_size: int = 128) -> int:
    return int(_load().gfx906_fa_amd_paged_attention_workspace_size(
        num_seqs, num_tokens, num_heads, num_kv_heads, head_size, max_query_len, max_seq_len))


def workspace_bound(max_num_seqs: int, max_num_tokens: int, num_heads: int, num_kv_heads: int,
                    head_size: int = 128) -> int:
    """Workspace bytes covering every ``paged_attention`` call with at most
    max_num_seqs sequences and max_num_tokens query tokens, whatever their
    query lengths and mix (decode, verify, prefill)."""
    return int(_load().gfx906_fa_amd_paged_attention_workspace_bound(
        int(max_num_seqs), int(max_num_tokens), num_heads, num_kv_heads, head_size))


def workspace_bound_info(max_num_seqs: int, max_num_tokens: int, num_heads: int, num_kv_heads: int,
                         max_seq_len: int = -1, head_size: int = 128) -> dict:
    """The workspace bound in its two parts: ``regions``, the bytes every
    call within the limits needs (its plan_info ``img_offset`` is at most
    this), and ``img_bytes``, the room for prefill tile images of contexts up
    to max_seq_len keys (-1: any context; the library's 1 GiB cap).  The
    image room is optional: with ``regions`` bytes every such call runs,
    dequantizing its own prefill tiles where images do not fit."""
    buf = (ctypes.c_int64 * 2)()
    n = _load().gfx906_fa_amd_paged_attention_workspace_bound_info(
        int(max_num_seqs), int(max_num_tokens), num_heads, num_kv_heads, head_size, int(max_seq_len), buf, 2)
    _check(n == 2, f"workspace_bound_info: invalid shape (returned {n})")
    return {"regions": int(buf[0]), "img_bytes": int(buf[1])}


PLAN_FIELDS = ("bytes", "decode_classes", "dec_rows_max", "prefill", "pf_items_max", "pf_grid_items",
               "pf_split_max", "pf_slots_max", "pf_header_offset", "cus", "img_offset", "img_bytes",
               "pf_rows")


def plan_info(num_seqs: int, num_tokens: int, num_heads: int, num_kv_heads: int, max_query_len: int,
              max_seq_len: int, head_size: int = 128) -> dict:
    """The launch plan of a call shape (see PLAN_FIELDS).  ``pf_header_offset``
    is where, in the workspace, the call leaves its prefill work-list header:
    int32 item count, int32 count of row tiles split over the keys, int32 1
    when the prefill tiles were dequantized once into the workspace as LDS
    images (else 0), int32 their count per kv head.  ``bytes`` (the
    workspace_size) is ``img_offset``, the regions every call needs, plus
    ``img_bytes`` of room for those images; a smaller workspace of at least
    ``img_offset`` bytes runs the same call with the prefill workgroups
    dequantizing every tile themselves.  ``pf_rows``: query rows per prefill
    row tile (256, or 128 for key-interleaved tiles; 0 without prefill)."""
    buf = (ctypes.c_int64 * len(PLAN_FIELDS))()
    n = _load().gfx906_fa_amd_paged_attention_plan_info(num_seqs, num_tokens, num_heads, num_kv_heads,
                                                         head_size, max_query_len, max_seq_len, buf,
                                                         len(PLAN_FIELDS))
    _check(n == len(PLAN_FIELDS), f"plan_info: invalid shape (returned {n})")
    return dict(zip(PLAN_FIELDS, (int(v) for v in buf)))


def device_cus() -> int:
    """CUs of the current device the plans target (256 without a device)."""
    return int(_load().gfx906_fa_amd_device_cus())


def stream_read(src: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Reads every byte of the contiguous device tensor ``src`` once (a
    read-only streaming ceiling for measurements) and returns the per-wave
    XOR words.  Not part of the reference interface."""
    _check(src.is_cuda and src.is_contiguous(), "stream_read: src must be a contiguous CUDA/HIP tensor")
    nw = int(_load().gfx906_fa_amd_stream_read_words())
    if out is None:
        out = torch.empty(nw, dtype=torch.int32, device=src.device)
    _check(out.is_cuda and out.numel() >= nw and out.element_size() == 4, "stream_read: out too small")
    err = _load().gfx906_fa_amd_stream_read(src.data_ptr(), src.numel() * src.element_size(), out.data_ptr(),
                                             out.numel(), _stream(src.device))
    _check(err == 0, f"stream_read failed ({err})")
    return out


def paged_attention(query: torch.Tensor, key_cache: torch.Tensor, value_cache: torch.Tensor,
                    block_table: torch.Tensor, seq_lens: torch.Tensor,
                    query_start_loc: torch.Tensor, max_query_len: int, max_seq_len: int,
                    scale: float, out: Optional[torch.Tensor] = None,
                    workspace: Optional[torch.Tensor] = None,
                    q_abs_offset: Optional[torch.Tensor] = None, causal: bool = True,
                    out_dtype: Optional[torch.dtype] = None, new_key: Optional[torch.Tensor] = None,
                    new_value: Optional[torch.Tensor] = None,
                    slot_mapping: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Varlen direct-paged attention: query [T, Hq, 128] -> out [T, Hq, 128].

    ``max_query_len`` / ``max_seq_len`` must bound the device values (they
    size the launch; they are host ints so no device sync is needed).
    With ``new_key`` / ``new_value`` [T, Hkv, 128] (the query dtype) and
    ``slot_mapping`` (int64 [T]) the step's K/V are first written to the cache
    as ``reshape_and_cache_q8_kv`` does; decode-shaped batches do it inside
    the attention launch."""
    for t, n in ((query, "query"), (block_table, "block_table"), (seq_lens, "seq_lens"),
                 (query_start_loc, "query_start_loc")):
        _cuda(t, n)
    _check(query.dtype in _DT, "query must be fp16, bf16 or fp32")
    _check(query.dim() == 3 and query.shape[2] == 128, "query must be [num_tokens, Hq, 128]")
    T, Hq, D = query.shape
    if T == 0:  # no query rows: nothing to compute or write (an empty tensor's strides are arbitrary)
        return out if out is not None else torch.empty((0, Hq, D), dtype=out_dtype or query.dtype,
                                                       device=query.device)
    _check(query.stride(2) == 1, "query rows must be contiguous")
    bs, Hkv, cbs, chs = _plane_info(key_cache, value_cache)
    _check(Hq % Hkv == 0, f"heads_q={Hq} must be divisible by heads_kv={Hkv}")
    _check(block_table.dtype == torch.int32 and block_table.dim() == 2 and block_table.stride(1) == 1,
           "block_table must be int32 [num_seqs, max_blocks] with contiguous rows")
    _check(seq_lens.dtype == torch.int32 and seq_lens.is_contiguous(), "seq_lens must be contiguous int32")
    _check(query_start_loc.dtype == torch.int32 and query_start_loc.is_contiguous(),
           "query_start_loc must be contiguous int32")
    B = seq_lens.shape[0]
    _check(block_table.shape[0] >= B and query_start_loc.shape[0] >= B + 1,
           "block_table / query_start_loc shorter than seq_lens")
    if q_abs_offset is not None:
        _cuda(q_abs_offset, "q_abs_offset")
        _check(q_abs_offset.dtype == torch.int32 and q_abs_offset.is_contiguous()
               and q_abs_offset.shape[0] >= B, "q_abs_offset must be int32 [B]")
    if out is None:
        out = torch.empty((T, Hq, D), dtype=out_dtype or query.dtype, device=query.device)
    _cuda(out, "out")
    _check(out.dtype in _DT and out.dim() == 3 and tuple(out.shape[1:]) == (Hq, D)
           and out.shape[0] >= T and out.stride(2) == 1, "out must be [num_tokens, Hq, 128] fp32/fp16/bf16")
    need = workspace_size(B, T, Hq, Hkv, max_query_len, max_seq_len)
    if workspace is None:
        workspace = new_workspace(need, query.device)
    elif workspace.numel() * workspace.element_size() < need:
        # the prefill tile-image room is optional: a workspace with the regions
        # every call needs runs as given (its prefill workgroups dequantize)
        have = workspace.numel() * workspace.element_size()
        if have < plan_info(B, T, Hq, Hkv, max_query_len, max_seq_len, D)["img_offset"]:
            workspace = new_workspace(need, query.device)
    _check(workspace.data_ptr() % 256 == 0, "workspace must be 256-byte aligned")
    ws_bytes = workspace.numel() * workspace.element_size()
    if new_key is not None or new_value is not None or slot_mapping is not None:
        _check(new_key is not None and new_value is not None and slot_mapping is not None,
               "new_key, new_value and slot_mapping go together")
        for t, n in ((new_key, "new_key"), (new_value, "new_value"), (slot_mapping, "slot_mapping")):
            _cuda(t, n)
        _check(new_key.dtype == query.dtype and new_value.dtype == query.dtype,
               "new_key / new_value must have the query dtype")
        _check(new_key.dim() == 3 and new_value.shape == new_key.shape and new_key.shape[0] >= T
               and tuple(new_key.shape[1:]) == (Hkv, D), "new_key / new_value must be [num_tokens, Hkv, 128]")
        _check(new_key.stride(2) == 1 and new_value.stride(2) == 1, "new_key / new_value rows must be contiguous")
        _check(slot_mapping.dtype == torch.int64 and slot_mapping.shape[0] >= T, "slot_mapping must be int64 [T]")
        sm = slot_mapping.contiguous()
        err = _load().gfx906_fa_amd_paged_attention_kv_write(
            _ptr(query), _DT[query.dtype], query.stride(0), query.stride(1), _ptr(key_cache),
            _ptr(value_cache), cbs, chs, _ptr(block_table), block_table.stride(0), _ptr(seq_lens),
            _ptr(query_start_loc), _ptr(q_abs_offset), 1 if causal else 0, B, T, Hq, Hkv, D, bs,
            int(max_query_len), int(max_seq_len), float(scale), _ptr(out), _DT[out.dtype],
            out.stride(0), out.stride(1), _ptr(workspace), ws_bytes, _ptr(new_key), _ptr(new_value),
            _DT[new_key.dtype], new_key.stride(0), new_key.stride(1), new_value.stride(0), new_value.stride(1),
            _ptr(sm), _stream(query.device))
        _ok(err, "gfx906_fa_amd_paged_attention_kv_write")
        return out
    err = _load().gfx906_fa_amd_paged_attention(
        _ptr(query), _DT[query.dtype], query.stride(0), query.stride(1), _ptr(key_cache),
        _ptr(value_cache), cbs, chs, _ptr(block_table), block_table.stride(0), _ptr(seq_lens),
        _ptr(query_start_loc), _ptr(q_abs_offset), 1 if causal else 0, B, T, Hq, Hkv, D, bs,
        int(max_query_len), int(max_seq_len), float(scale), _ptr(out), _DT[out.dtype],
        out.stride(0), out.stride(1), _ptr(workspace), ws_bytes,
        _stream(query.device))
    _ok(err, "gfx906_fa_amd_paged_attention")
    return out


def _mask_args(mask: Optional[torch.Tensor], B: int, Sq: int, q_abs_offset):
    """fp16 additive mask [B, Sq, Skv_pad] (``extension/gfx906_fa.cpp:214-227``)
    -> (tensor, batch stride, row stride, columns) for the tiled entry."""
    if mask is None:
        return None, 0, 0, 0
    _check(q_abs_offset is None,
           "q_abs_offset and mask are mutually exclusive (inline causal replaces mask)")
    _cuda(mask, "mask")
    _check(mask.dtype == torch.float16, "mask must be fp16")
    _check(mask.dim() == 3, "mask must be 3D [B, Sq, Skv_pad]")
    _check(mask.shape[0] == B, "mask.size(0) must equal batch")
    _check(mask.shape[1] == Sq, "mask.size(1) must equal seq_q")
    m = mask.contiguous()
    return m, m.stride(0), m.stride(1), m.shape[2]


def forward(q: torch.Tensor, k_q8: torch.Tensor, v_fp16: torch.Tensor, scale: float,
            kv_max: Optional[torch.Tensor] = None, mask: Optional[torch.Tensor] = None,
            q_abs_offset: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Contiguous attention with the reference signature
    (``extension/gfx906_fa.cpp:120-265``, bound at 662-666):
    q fp32 [B, Hq, Sq, D], k_q8 uint8 [B, Hkv, Skv, D/32*34] (AoS Q8_0 rows),
    v_fp16 fp16 [B, Hkv, Skv, D] -> fp32 [B, Hq, Sq, D].  K is dequantized,
    V stays fp16, softmax in fp32.  kv_max int32 [B]: every row sees keys
    < kv_max[b]; q_abs_offset int32 [B]: row j sees keys
    k <= q_abs_offset[b] + j (inline causal, ``kernel/fattn-q8.cuh:646-653``);
    mask fp16 [B, Sq, Skv_pad]: added to the scaled scores
    (``kernel/fattn-q8.cuh:643-644``), exclusive with q_abs_offset.  D = 128
    only, as the reference launcher (``extension/gfx906_fa_launcher.cu:76-79``).

    Decode shapes (Sq * Hq / Hkv <= 16 rows per kv-head, no mask) read K and
    V in these layouts directly, split over the keys across the device
    (gfx906_fa_amd_flat_decode); other shapes repack K and V into the planar
    sub-pages once per call and run the tiled prefill kernel."""
    for t, n in ((q, "q"), (k_q8, "k_q8"), (v_fp16, "v_fp16")):
        _cuda(t, n)
        _check(t.is_contiguous(), f"{n} must be contiguous")
    _check(q.dtype == torch.float32, "q must be fp32")
    _check(k_q8.dtype == torch.uint8, "k_q8 must be uint8 (block_q8_0 bytes)")
    _check(v_fp16.dtype == torch.float16, "v_fp16 must be fp16")
    _check(q.dim() == 4, "q must be 4D [B, Hq, Sq, D]")
    _check(v_fp16.dim() == 4, "v_fp16 must be 4D [B, Hkv, Skv, D]")
    B, Hq, Sq, D = q.shape
    Hkv, Skv = v_fp16.shape[1], v_fp16.shape[2]
    _check(v_fp16.shape[0] == B, "v batch mismatch")
    _check(v_fp16.shape[3] == D, "v head_dim mismatch")
    _check(D % QK8_0 == 0, "head_dim must be multiple of 32")
    _check(k_q8.dim() == 4 and tuple(k_q8.shape[:3]) == (B, Hkv, Skv),
           "k_q8 first 3 dims must match [B, Hkv, Skv]")
    _check(k_q8.shape[3] == D // QK8_0 * Q8_0_BYTES, "k_q8 last dim = (D/32)*34 bytes")
    _check(D == 128, f"head_dim={D} unsupported (only 128)")
    _check(Hq % Hkv == 0, f"heads_q={Hq} must be divisible by heads_kv={Hkv}")
    _check(mask is None or mask.dim() != 3 or mask.shape[2] >= Skv, "mask.size(2) must be >= seq_kv")
    mk, mbs, mrs, mcols = _mask_args(mask, B, Sq, q_abs_offset)
    dev = q.device
    out = torch.empty((B * Sq, Hq, D), dtype=torch.float32, device=dev)
    if B == 0 or Sq == 0 or Hq == 0:
        return out.view(B, Sq, Hq, D).transpose(1, 2).contiguous()
    if kv_max is not None:
        _cuda(kv_max, "kv_max")
        _check(kv_max.dtype == torch.int32, "kv_max must be int32")
        _check(kv_max.dim() == 1 and kv_max.shape[0] == B, "kv_max must be 1D [B]")
        sl = kv_max.clamp(0, Skv).to(torch.int32).contiguous()
    else:
        sl = torch.full((B,), Skv, dtype=torch.int32, device=dev)
    if q_abs_offset is not None:
        _cuda(q_abs_offset, "q_abs_offset")
        _check(q_abs_offset.dtype == torch.int32 and q_abs_offset.dim() == 1 and q_abs_offset.shape[0] == B,
               "q_abs_offset must be 1D [B]")
        q_abs_offset = q_abs_offset.contiguous()
    L = _load()
    st = _stream(dev)
    if mask is None and Sq * (Hq // Hkv) <= 16 and Skv > 0:
        # decode shapes: the contiguous layouts read as they are, split over the keys
        q_bshd = q.transpose(1, 2).contiguous().view(B * Sq, Hq, D)
        ws = new_workspace(L.gfx906_fa_amd_flat_decode_workspace_size(B, Sq, Hq, Hkv, Skv), dev)
        _ok(L.gfx906_fa_amd_flat_decode(_ptr(q_bshd), _DT[torch.float32], q_bshd.stride(0), q_bshd.stride(1),
                                         _ptr(k_q8), _ptr(v_fp16), _ptr(sl), _ptr(q_abs_offset), B, Sq, Hq, Hkv,
                                         Skv, D, float(scale), _ptr(out), out.stride(0), out.stride(1),
                                         _ptr(ws), ws.numel(), st), "gfx906_fa_amd_flat_decode")
        return out.view(B, Sq, Hq, D).transpose(1, 2).contiguous()
    skp = (max(Skv, 1) + SUBPAGE_TOKENS - 1) // SUBPAGE_TOKENS
    kp = torch.empty((B, Hkv, skp * SUBPAGE_BYTES), dtype=torch.uint8, device=dev)
    vp = torch.empty((B, Hkv, skp * 4096), dtype=torch.uint8, device=dev)
    if Skv > 0:
        _ok(L.gfx906_fa_amd_pack_flat_kv(_ptr(k_q8), _ptr(v_fp16), _ptr(kp), _ptr(vp), B * Hkv, Skv, D, st),
            "gfx906_fa_amd_pack_flat_kv")
    else:
        kp.zero_()
        vp.zero_()
    bt = torch.arange(B, dtype=torch.int32, device=dev).view(B, 1)
    qsl = torch.arange(0, (B + 1) * Sq, Sq, dtype=torch.int32, device=dev)
    q_bshd = q.transpose(1, 2).contiguous().view(B * Sq, Hq, D)
    err = L.gfx906_fa_amd_paged_attention_tiled(
        _ptr(q_bshd), _DT[torch.float32], q_bshd.stride(0), q_bshd.stride(1), _ptr(kp), _ptr(vp), 1,
        kp.stride(0), kp.stride(1), vp.stride(0), vp.stride(1), _ptr(bt), 1, _ptr(sl), _ptr(qsl),
        _ptr(q_abs_offset), 1 if q_abs_offset is not None else 0, _ptr(mk), mbs, mrs, mcols,
        B, B * Sq, Hq, Hkv, D, skp * SUBPAGE_TOKENS, Sq, float(scale), _ptr(out), out.stride(0),
        out.stride(1), st)
    _ok(err, "gfx906_fa_amd_paged_attention_tiled")
    return out.view(B, Sq, Hq, D).transpose(1, 2).contiguous()


def forward_paged_direct(q: torch.Tensor, key_cache_q8: torch.Tensor, value_cache: torch.Tensor,
                         block_table: torch.Tensor, seq_lens: torch.Tensor, scale: float,
                         mask: Optional[torch.Tensor] = None,
                         q_abs_offset: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Padded-batch entry with the reference signature
    (``extension/gfx906_fa.cpp:516-658``): q [B, Hq, Sq, D] -> fp32
    [B, Hq, Sq, D].  key_cache_q8 / value_cache are the planar K and V planes
    of this backend (V is Q8_0 too).  Without q_abs_offset every row sees all
    seq_lens[b] keys (``kv_max`` cutoff); with it, row j sees keys
    k <= q_abs_offset[b] + j (inline causal, ``kernel/fattn-q8.cuh:646-653``).
    mask fp16 [B, Sq, Skv_pad] is added to the scaled scores
    (``kernel/fattn-q8.cuh:643-644``); exclusive with q_abs_offset."""
    _cuda(q, "q")
    _check(q.dim() == 4, "q must be 4D [B, Hq, Sq, D]")
    B, Hq, Sq, D = q.shape
    _check(block_table.shape[0] == B, "block_table[0] must equal batch")
    _check(seq_lens.dim() == 1 and seq_lens.shape[0] == B, "seq_lens must be [batch]")
    q_bshd = q.transpose(1, 2).reshape(B * Sq, Hq, D)
    qsl = torch.arange(0, (B + 1) * Sq, Sq, dtype=torch.int32, device=q.device)
    bt = block_table if block_table.dtype == torch.int32 else block_table.to(torch.int32)
    sl = seq_lens if seq_lens.dtype == torch.int32 else seq_lens.to(torch.int32)
    max_kv = bt.shape[1] * (key_cache_q8.shape[2] // SUBPAGE_BYTES * SUBPAGE_TOKENS)
    if mask is None:
        out = paged_attention(q_bshd, key_cache_q8, value_cache, bt.contiguous(), sl.contiguous(), qsl,
                              Sq, max_kv, scale, q_abs_offset=q_abs_offset,
                              causal=q_abs_offset is not None, out_dtype=torch.float32)
        return out.view(B, Sq, Hq, D).transpose(1, 2).contiguous()
    # materialised mask: the tiled kernel over the same planar Q8 planes
    mk, mbs, mrs, mcols = _mask_args(mask, B, Sq, q_abs_offset)
    q_bshd = q_bshd.contiguous()
    sl = sl.contiguous()
    _check(q_bshd.dtype in _DT, "q must be fp32, fp16 or bf16")
    bs, Hkv, cbs, chs = _plane_info(key_cache_q8, value_cache)
    _check(Hq % Hkv == 0, f"heads_q={Hq} must be divisible by heads_kv={Hkv}")
    out = torch.empty((B * Sq, Hq, D), dtype=torch.float32, device=q.device)
    bt = bt.contiguous()
    err = _load().gfx906_fa_amd_paged_attention_tiled(
        _ptr(q_bshd), _DT[q_bshd.dtype], q_bshd.stride(0), q_bshd.stride(1), _ptr(key_cache_q8),
        _ptr(value_cache), 0, cbs, chs, cbs, chs, _ptr(bt), bt.stride(0), _ptr(sl),
        _ptr(qsl), None, 0, _ptr(mk), mbs, mrs, mcols, B, B * Sq, Hq, Hkv, D, bs, Sq, float(scale),
        _ptr(out), out.stride(0), out.stride(1), _stream(q.device))
    _ok(err, "gfx906_fa_amd_paged_attention_tiled")
    return out.view(B, Sq, Hq, D).transpose(1, 2).contiguous()


# ---------------------------------------------------------------------------
# PyTorch custom ops: torch.ops.gfx906_fa.*
# ---------------------------------------------------------------------------
# The ops above as torch.library custom ops, so torch.compile / torch.export
# trace them as opaque nodes (the reference registers its ops through a torch
# extension module, extension/gfx906_fa.cpp:660-690).  Each op runs the
# function of the same name above; a fake implementation gives the output
# shapes for tracing.  Custom ops may not return an alias of an input, so the
# ops that can write into caller buffers come in a functional form (outputs
# allocated) and an ``_out`` form (outputs written in place, nothing returned).
# In-place arguments are declared in each schema: caches, workspaces, outputs
# and the query / key the fused rotary write rotates.  An in-place argument
# that may be None (the workspace) has no default: torch's in-place
# bookkeeping indexes it positionally, so callers pass it, None included.
_NS = "gfx906_fa"


def _register_torch_ops() -> None:
    from torch.library import custom_op

    @custom_op(f"{_NS}::quantize_q8_0", mutates_args=())
    def _quantize_q8_0(k_fp16: torch.Tensor) -> torch.Tensor:
        return quantize_q8_0(k_fp16)

    @_quantize_q8_0.register_fake
    def _(k_fp16):
        D = k_fp16.shape[-1]
        return k_fp16.new_empty((*k_fp16.shape[:-1], D // QK8_0 * Q8_0_BYTES), dtype=torch.uint8)

    @custom_op(f"{_NS}::reshape_and_cache_q8", mutates_args=("k_cache_q8",))
    def _reshape_and_cache_q8(key: torch.Tensor, slot_mapping: torch.Tensor, k_cache_q8: torch.Tensor) -> None:
        reshape_and_cache_q8(key, slot_mapping, k_cache_q8)

    @_reshape_and_cache_q8.register_fake
    def _(key, slot_mapping, k_cache_q8):
        return None

    def _gather_shapes(key_cache_q8, value_cache, block_table, Sk):
        B = block_table.shape[0]
        _, _, Hkv, bpr = key_cache_q8.shape
        return (B, Hkv, Sk, bpr), (B, Hkv, Sk, value_cache.shape[3])

    @custom_op(f"{_NS}::gather_paged_kv_q8", mutates_args=())
    def _gather_paged_kv_q8(key_cache_q8: torch.Tensor, value_cache: torch.Tensor, block_table: torch.Tensor,
                            seq_lens: torch.Tensor, Sk: int) -> tuple[torch.Tensor, torch.Tensor]:
        k, v = gather_paged_kv_q8(key_cache_q8, value_cache, block_table, seq_lens, Sk)
        return k, v

    @_gather_paged_kv_q8.register_fake
    def _(key_cache_q8, value_cache, block_table, seq_lens, Sk):
        ks, vs = _gather_shapes(key_cache_q8, value_cache, block_table, Sk)
        return key_cache_q8.new_empty(ks), value_cache.new_empty(vs)

    @custom_op(f"{_NS}::gather_paged_kv_q8_out", mutates_args=("k_out", "v_out"))
    def _gather_paged_kv_q8_out(key_cache_q8: torch.Tensor, value_cache: torch.Tensor, block_table: torch.Tensor,
                                seq_lens: torch.Tensor, Sk: int, k_out: torch.Tensor, v_out: torch.Tensor) -> None:
        k, v = gather_paged_kv_q8(key_cache_q8, value_cache, block_table, seq_lens, Sk, k_out, v_out)
        _check(k.data_ptr() == k_out.data_ptr() and v.data_ptr() == v_out.data_ptr(),
               "gather_paged_kv_q8_out: k_out / v_out must be contiguous [B, Hkv, Sk, row] of the cache dtypes")

    @_gather_paged_kv_q8_out.register_fake
    def _(key_cache_q8, value_cache, block_table, seq_lens, Sk, k_out, v_out):
        return None

    @custom_op(f"{_NS}::forward", mutates_args=())
    def _forward(q: torch.Tensor, k_q8: torch.Tensor, v_fp16: torch.Tensor, scale: float, kv_max: Optional[torch.Tensor] = None,
                 mask: Optional[torch.Tensor] = None, q_abs_offset: Optional[torch.Tensor] = None) -> torch.Tensor:
        return forward(q, k_q8, v_fp16, scale, kv_max, mask, q_abs_offset)

    @_forward.register_fake
    def _(q, k_q8, v_fp16, scale, kv_max=None, mask=None, q_abs_offset=None):
        return q.new_empty(q.shape, dtype=torch.float32)

    @custom_op(f"{_NS}::forward_paged_direct", mutates_args=())
    def _forward_paged_direct(q: torch.Tensor, key_cache_q8: torch.Tensor, value_cache: torch.Tensor, block_table: torch.Tensor,
                              seq_lens: torch.Tensor, scale: float, mask: Optional[torch.Tensor] = None,
                              q_abs_offset: Optional[torch.Tensor] = None) -> torch.Tensor:
        return forward_paged_direct(q, key_cache_q8, value_cache, block_table, seq_lens, scale, mask,
                                    q_abs_offset)

    @_forward_paged_direct.register_fake
    def _(q, key_cache_q8, value_cache, block_table, seq_lens, scale, mask=None, q_abs_offset=None):
        return q.new_empty(q.shape, dtype=torch.float32)

    @custom_op(f"{_NS}::reshape_and_cache_q8_kv", mutates_args=("key_cache", "value_cache"))
    def _reshape_and_cache_q8_kv(key: torch.Tensor, value: torch.Tensor, slot_mapping: torch.Tensor, key_cache: torch.Tensor,
                                 value_cache: torch.Tensor) -> None:
        reshape_and_cache_q8_kv(key, value, slot_mapping, key_cache, value_cache)

    @_reshape_and_cache_q8_kv.register_fake
    def _(key, value, slot_mapping, key_cache, value_cache):
        return None

    @custom_op(f"{_NS}::rope_and_cache_q8_kv", mutates_args=("query", "key", "key_cache", "value_cache"))
    def _rope_and_cache_q8_kv(positions: torch.Tensor, query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                              cos_sin_cache: torch.Tensor, is_neox: bool, slot_mapping: torch.Tensor, key_cache: torch.Tensor,
                              value_cache: torch.Tensor, rot_dim: Optional[int] = None) -> None:
        rope_and_cache_q8_kv(positions, query, key, value, cos_sin_cache, is_neox, slot_mapping, key_cache,
                             value_cache, rot_dim)

    @_rope_and_cache_q8_kv.register_fake
    def _(positions, query, key, value, cos_sin_cache, is_neox, slot_mapping, key_cache, value_cache,
          rot_dim=None):
        return None

    @custom_op(f"{_NS}::gather_paged_kv_q8q8", mutates_args=())
    def _gather_paged_kv_q8q8(key_cache: torch.Tensor, value_cache: torch.Tensor, block_table: torch.Tensor, seq_lens: torch.Tensor,
                              Sk: int) -> tuple[torch.Tensor, torch.Tensor]:
        k, v = gather_paged_kv_q8q8(key_cache, value_cache, block_table, seq_lens, Sk)
        return k, v

    @_gather_paged_kv_q8q8.register_fake
    def _(key_cache, value_cache, block_table, seq_lens, Sk):
        shape = (block_table.shape[0], key_cache.shape[1], Sk, 136)
        return key_cache.new_empty(shape), key_cache.new_empty(shape)

    @custom_op(f"{_NS}::paged_attention", mutates_args=("workspace",))
    def _paged_attention(query: torch.Tensor, key_cache: torch.Tensor, value_cache: torch.Tensor, block_table: torch.Tensor,
                         seq_lens: torch.Tensor, query_start_loc: torch.Tensor, max_query_len: int, max_seq_len: int,
                         scale: float, workspace: Optional[torch.Tensor],
                         q_abs_offset: Optional[torch.Tensor] = None, causal: bool = True,
                         out_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
        return paged_attention(query, key_cache, value_cache, block_table, seq_lens, query_start_loc,
                               max_query_len, max_seq_len, scale, workspace=workspace,
                               q_abs_offset=q_abs_offset, causal=causal, out_dtype=out_dtype)

    @_paged_attention.register_fake
    def _(query, key_cache, value_cache, block_table, seq_lens, query_start_loc, max_query_len, max_seq_len,
          scale, workspace, q_abs_offset=None, causal=True, out_dtype=None):
        return query.new_empty(query.shape, dtype=out_dtype or query.dtype)

    @custom_op(f"{_NS}::paged_attention_out",
               mutates_args=("out", "workspace", "key_cache", "value_cache"))
    def _paged_attention_out(query: torch.Tensor, key_cache: torch.Tensor, value_cache: torch.Tensor, block_table: torch.Tensor,
                             seq_lens: torch.Tensor, query_start_loc: torch.Tensor, max_query_len: int, max_seq_len: int,
                             scale: float, out: torch.Tensor, workspace: Optional[torch.Tensor],
                             q_abs_offset: Optional[torch.Tensor] = None, causal: bool = True,
                             new_key: Optional[torch.Tensor] = None, new_value: Optional[torch.Tensor] = None,
                             slot_mapping: Optional[torch.Tensor] = None) -> None:
        """The backend's step: attention into ``out`` (the model dtype), with
        the step's K/V written to the cache first when new_key / new_value /
        slot_mapping are given (the caches are in-place arguments for that)."""
        # the regions every call needs; the tile-image room past them is
        # optional (without it the prefill workgroups dequantize their tiles)
        need = plan_info(seq_lens.shape[0], query.shape[0], query.shape[1], key_cache.shape[1],
                         max_query_len, max_seq_len, query.shape[2])["img_offset"]
        _check(workspace is None or workspace.numel() * workspace.element_size() >= need,
               f"paged_attention_out: workspace needs {need} bytes")
        paged_attention(query, key_cache, value_cache, block_table, seq_lens, query_start_loc, max_query_len,
                        max_seq_len, scale, out=out, workspace=workspace, q_abs_offset=q_abs_offset,
                        causal=causal, new_key=new_key, new_value=new_value, slot_mapping=slot_mapping)

    @_paged_attention_out.register_fake
    def _(query, key_cache, value_cache, block_table, seq_lens, query_start_loc, max_query_len, max_seq_len,
          scale, out, workspace, q_abs_offset=None, causal=True, new_key=None, new_value=None,
          slot_mapping=None):
        return None


TORCH_OPS = ("quantize_q8_0", "reshape_and_cache_q8", "gather_paged_kv_q8", "gather_paged_kv_q8_out",
             "forward", "forward_paged_direct", "reshape_and_cache_q8_kv", "rope_and_cache_q8_kv",
             "gather_paged_kv_q8q8", "paged_attention", "paged_attention_out")

_load()
if not hasattr(torch.ops, _NS) or not hasattr(getattr(torch.ops, _NS), "paged_attention"):
    _register_torch_ops()
