"""GPU: the contiguous decode path of ``gfx906_fa.forward``.

Decode shapes (Sq * Hq / Hkv <= 16 rows per kv-head, no mask) read the
reference's contiguous layouts directly (AoS Q8_0 K rows, fp16 V rows; the
reference's ``extension/gfx906_fa.cpp:120-265`` contract) and are split over
the keys into single-wave pieces merged by a second launch.  Checked against
``oracle.flat_attention_ref``: the reference benchmark's decode shapes
(``tests/bench.py:39-66``: 8/4 and 48/8 heads, one query), key counts around
the 16-token sub-page and piece boundaries (1, 15, 16, 17, 129, ...), batches
whose (batch, kv-head) segments start 8 bytes past a 16-byte boundary (odd
Skv), kv_max (including 0 keys), q_abs_offset (inline causal), 16 rows, and
a 128K-key decode; and whether the call split its keys (workspace size)."""
import numpy as np
import pytest
import torch

import gfx906_fa
from gpu_common import announce, assert_close, need_gpu
from oracle import q8_oracle as O

DEV = "cuda"
pytestmark = pytest.mark.gpu


def _inputs(seed, B, Hq, Hkv, Sq, Skv):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((B, Hq, Sq, 128)).astype(np.float32)
    k = rng.standard_normal((B, Hkv, Skv, 128)).astype(np.float16)
    v = rng.standard_normal((B, Hkv, Skv, 128)).astype(np.float16)
    return q, O.quantize_q8_0_rows(k), v


CASES = [
    # name, B, Hq, Hkv, Sq, Skv, kv_max, q_abs
    ("dec_1", 1, 8, 4, 1, 1, None, None),
    ("dec_15", 1, 8, 4, 1, 15, None, None),
    ("dec_16", 1, 8, 4, 1, 16, None, None),
    ("dec_17_b3", 3, 8, 4, 1, 17, None, None),
    ("dec_128", 1, 8, 4, 1, 128, None, None),
    ("dec_129_b2", 2, 8, 4, 1, 129, None, None),
    ("dec_1000_odd_b3", 3, 8, 2, 1, 1001, None, None),
    ("dec_4096", 1, 8, 4, 1, 4096, None, None),
    ("dec_16383", 1, 8, 4, 1, 16383, None, None),
    ("mmx_dec_1k", 1, 48, 8, 1, 1024, None, None),
    ("mmx_dec_8k_odd", 1, 48, 8, 1, 8191, None, None),
    ("kvmax_b4", 4, 8, 2, 1, 3001, [3001, 17, 0, 2048], None),
    ("causal_sq2_g8", 2, 16, 2, 2, 2000, None, [1998, 1000]),
    ("causal_sq16_g1", 1, 4, 4, 16, 777, [700], [684]),
    ("sq4_g4_b2", 2, 16, 4, 4, 5000, None, None),
]


def _run(q, kq, v, scale, kvm, qa):
    return gfx906_fa.forward(torch.from_numpy(q).to(DEV), torch.from_numpy(kq).to(DEV), torch.from_numpy(v).to(DEV),
                             scale, kv_max=None if kvm is None else torch.from_numpy(kvm).to(DEV),
                             q_abs_offset=None if qa is None else torch.from_numpy(qa).to(DEV))


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_flat_decode_matches_oracle(case):
    need_gpu()
    name, B, Hq, Hkv, Sq, Skv, kv_max, q_abs = case
    announce(f"flat decode {name}")
    assert Sq * (Hq // Hkv) <= 16
    q, kq, v = _inputs(sum(map(ord, name)), B, Hq, Hkv, Sq, Skv)
    kvm = None if kv_max is None else np.asarray(kv_max, np.int32)
    qa = None if q_abs is None else np.asarray(q_abs, np.int32)
    scale = 1.0 / np.sqrt(128)
    out = _run(q, kq, v, scale, kvm, qa)
    torch.cuda.synchronize()
    assert out.shape == (B, Hq, Sq, 128) and out.dtype == torch.float32
    assert_close(out.cpu().numpy(), O.flat_attention_ref(q, kq, v, scale, kv_max=kvm, q_abs_offset=qa))


def test_flat_decode_splits_long_contexts():
    """Short contexts run one workgroup per (batch, kv-head) and write the
    output directly (no partials); long ones are split over the keys."""
    need_gpu()
    L = gfx906_fa.lib()
    assert L.gfx906_fa_amd_flat_decode_workspace_size(1, 1, 8, 4, 128) == 256      # 8 sub-pages: whole
    big = L.gfx906_fa_amd_flat_decode_workspace_size(1, 1, 8, 4, 131072)
    pieces = big // (4 * 2 * 132 * 4)
    assert pieces >= 64, pieces                                                      # split for the device


def test_flat_decode_128k():
    """The reference benchmark's longest decode (8/4 heads, 131072 keys), one
    query, against the oracle."""
    need_gpu()
    announce("flat decode 128K 8/4")
    q, kq, v = _inputs(5, 1, 8, 4, 1, 131072)
    scale = 1.0 / np.sqrt(128)
    out = _run(q, kq, v, scale, None, None)
    torch.cuda.synchronize()
    assert_close(out.cpu().numpy(), O.flat_attention_ref(q, kq, v, scale))


def test_flat_decode_repeated_calls_are_identical():
    """The split and the merge are deterministic: two calls give the same
    bits (the workspace carries nothing between calls)."""
    need_gpu()
    announce("flat decode determinism")
    q, kq, v = _inputs(6, 2, 48, 8, 1, 9000)
    a = _run(q, kq, v, 0.088, None, None)
    b = _run(q, kq, v, 0.088, None, None)
    torch.cuda.synchronize()
    assert torch.equal(a, b)
