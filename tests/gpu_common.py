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


def seq_head_kv(b, s, h):
    """Dequantized K, V float32 [seq_len, 128] of sequence s, kv-head h, read
    from the GPU-written planar cache (whose bytes are checked separately):
    only that sequence's pages and that head's planes are copied."""
    sl = int(b.seq_lens[s])
    bs = b.block_size
    npg = max((sl + bs - 1) // bs, 1)
    pages = torch.from_numpy(b.block_table_np[s, :npg].astype(np.int64)).to(b.kv_cache.device)
    sub = b.kv_cache.index_select(0, pages)[:, :, h:h + 1].cpu().numpy()
    kh, vh = O.planar_dequant(np.ascontiguousarray(sub))
    return kh.reshape(npg * bs, 128)[:sl], vh.reshape(npg * bs, 128)[:sl]


def batch_oracle(b, rows=None, q_abs=None, causal=True):
    """float64 oracle output [T, Hq, D] for a workloads.Batch, computed from
    the GPU-written planar cache, one (sequence, kv-head) at a time.
    rows: optional list of query token indices to restrict the work (the
    others are left 0).  Row j of sequence s sees keys k < seq_len with
    k <= q_abs[s] + j when causal (q_abs defaults to seq_len - n_q)."""
    q = to_np_f32(b.query)
    qsl = b.qsl
    G = b.Hq // b.Hkv
    out = np.zeros(q.shape, np.float64)
    toks = np.arange(b.num_tokens) if rows is None else np.asarray(sorted(set(int(r) for r in rows)))
    seq_of = np.searchsorted(qsl, toks, side="right") - 1
    for s in np.unique(seq_of):
        s = int(s)
        ts = toks[seq_of == s]
        sl = int(b.seq_lens[s])
        nq = int(qsl[s + 1] - qsl[s])
        if sl <= 0:
            continue
        j = ts - int(qsl[s])
        qa = sl - nq if q_abs is None else int(q_abs[s])
        lim = np.minimum(qa + j, sl - 1) if causal else np.full(len(ts), sl - 1)
        for h in range(b.Hkv):
            K, V = seq_head_kv(b, s, h)
            out[ts, h * G:(h + 1) * G] = O.attention_rows_ref(q[ts, h * G:(h + 1) * G], K, V, lim, b.scale)
    return out
