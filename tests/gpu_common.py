"""Shared helpers for the ``gpu``-marked tests (parity against the CPU oracle)."""
import ctypes
import os
import sys

import numpy as np
import pytest
import torch

from oracle import q8_oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF_LIB = os.path.join(ROOT, "oracle", "_ref", "libref_q8_gfx950.so")

ATOL = 2e-3      # max-abs 2e-3 ...
RTOL_NORM = 1e-2  # ... and relative (Frobenius) error 1e-2


def need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


def announce(msg: str) -> None:
    """Names the case before a GPU step (a faulting run keeps only the tail)."""
    print(f"[gpu-case] {msg}", flush=True)
    sys.stdout.flush()


def to_np_f32(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy()


def host_bits(t: torch.Tensor) -> np.ndarray:
    """fp16 -> numpy float16; bf16 -> uint16 bit pattern; fp32 -> float32."""
    t = t.detach().cpu()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def assert_close(out: np.ndarray, ref: np.ndarray, atol=ATOL, rtol_norm=RTOL_NORM, extra=0.0):
    out = np.asarray(out, np.float64)
    ref = np.asarray(ref, np.float64)
    assert np.all(np.isfinite(out)), "non-finite output"
    err = np.abs(out - ref)
    bound = atol + extra * np.abs(ref)
    worst = np.unravel_index(np.argmax(err - bound), err.shape)
    assert np.all(err <= bound), f"max-abs {err.max():.3e} at {worst} (bound {bound[worst]:.3e})"
    den = np.linalg.norm(ref)
    if den > 0:
        assert np.linalg.norm(out - ref) / den <= rtol_norm


def ref_lib():
    """The reference's own quant kernels built from its sources for gfx950
    (oracle/Makefile); None when not built."""
    if not os.path.exists(REF_LIB):
        return None
    L = ctypes.CDLL(REF_LIB)
    P, I, I64 = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64
    L.launch_quantize_q8_0_dense.argtypes = [P, P, I, I, P]
    L.launch_quantize_q8_0_dense.restype = I
    L.launch_reshape_and_cache_q8.argtypes = [P, P, P, I, I, I, I, I64, I64, I64, I64, I64, P]
    L.launch_reshape_and_cache_q8.restype = I
    return L


def stream_ptr():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def batch_oracle(b, rows=None):
    """float64 oracle output [T, Hq, D] for a workloads.Batch, computed from
    the GPU-written planar cache (whose bytes are checked separately), only
    over the pages the batch references.  rows: optional list of query
    token indices to restrict the work (others left 0)."""
    bt = b.block_table_np
    q = to_np_f32(b.query)
    qsl = b.qsl

    def pages_of(seqs):
        """Dequantized sub-cache holding only the pages of `seqs`, and the
        remapped block table."""
        sel = bt[seqs]
        used = np.unique(sel[sel >= 0])
        idx = torch.from_numpy(used).to(b.kv_cache.device)
        sub = b.kv_cache.index_select(0, idx).cpu().numpy()
        remap = np.full(b.num_blocks, -1, np.int64)
        remap[used] = np.arange(len(used))
        kh, vh = O.planar_dequant(sub)
        return kh, vh, np.where(sel >= 0, remap[np.maximum(sel, 0)], -1).astype(np.int32)

    if rows is None:
        kh, vh, bt2 = pages_of(np.arange(b.num_seqs))
        return O.paged_attention_ref(q, kh, vh, bt2, b.seq_lens, qsl, b.scale)
    out = np.zeros(q.shape, np.float64)
    for tkn in rows:
        s = int(np.searchsorted(qsl, tkn, side="right") - 1)
        j = tkn - int(qsl[s])
        nq = int(qsl[s + 1] - qsl[s])
        sl = int(b.seq_lens[s])
        kh, vh, bt2 = pages_of(np.array([s]))
        # one-row sequence ending at the row's causal limit
        lim = sl - nq + j + 1
        o = O.paged_attention_ref(q[tkn:tkn + 1], kh, vh, bt2, np.array([lim], np.int32),
                                  np.array([0, 1], np.int32), b.scale)
        out[tkn] = o[0]
    return out
