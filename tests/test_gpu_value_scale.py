"""GPU: values far from unit scale.

The prefill kernel dequantizes V into fp16 (V^ = fp16(q * d_v), one rounding,
relative error at most 2^-12 of |v^|), while the decode kernel feeds V's int8
values to the matrix cores exactly and folds d_v into P.  A query row that
sees a single key outputs that key's V^ itself, so the prefill's error grows
with |v^|: the bound checked here is 2e-3 * max(1, max|v^| / 4), i.e. the
2e-3 absolute tolerance up to |v^| = 4 and 1/2000 of the largest value
beyond (above the 1/4096 rounding bound).  Values are drawn at 8x and 32x
N(0, 1) for fresh causal prompts (whose first rows see one and two keys),
prefix-cached chunks on 128- and 256-row tiles, and decode rows beside
them.  Both kernels also round K^ = fp16(q * d_k) (relative 2^-12 per
element), which moves every score by up to about 2^-11 of its own size; with
K at 4x N(0, 1) the scores, and so that error in the softmax weights, grow
4x, and the bound scales by max(1, max|k^| / 4) as well (measured at 4x:
2.5e-2 against 1.9e-2 for the value scale alone)."""
import numpy as np
import pytest
import torch

import gfx906_fa_workloads as W
from gpu_common import announce, assert_close, batch_oracle, need_gpu, to_np_f32

pytestmark = pytest.mark.gpu

CASES = [
    # name, seq_lens, q_lens, Hq, Hkv, v scale, k scale
    ("fresh300_v8", [300], [300], 8, 8, 8.0, 1.0),
    ("fresh2048_v32_48x8", [2048], [2048], 48, 8, 32.0, 1.0),
    ("chunk12_ctx3k_v8", [3000 + 12], [12], 48, 8, 8.0, 1.0),
    ("chunk500_ctx2k_v8", [2000 + 500], [500], 48, 8, 8.0, 1.0),
    ("mixed_decode_v8", [4000, 1500 + 200, 700, 9000 + 5], [1, 200, 1, 5], 48, 8, 8.0, 1.0),
    ("fresh600_v8_k4", [600], [600], 16, 4, 8.0, 4.0),
]


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_large_values_within_scaled_bound(case):
    need_gpu()
    name, sls, qls, Hq, Hkv, vs, ks = case
    announce(f"value scale {name}")
    b = W.build_batch(sls, qls, Hq, Hkv, seed=sum(map(ord, name)), write_cache=False)
    b.value = (b.value.float() * vs).to(b.value.dtype)
    b.key = (b.key.float() * ks).to(b.key.dtype)
    kp, vp = b.planes()
    import gfx906_fa
    gfx906_fa.reshape_and_cache_q8_kv(b.key, b.value, b.slot_mapping, kp, vp)
    out = W.attention(b, out_dtype=torch.float32)
    torch.cuda.synchronize()
    rows = None
    if b.num_tokens > 400:
        rng = np.random.default_rng(7)
        rows = sorted(set(rng.choice(b.num_tokens, 64, replace=False).tolist()) | {0, 1, 2, b.num_tokens - 1})
    ref = batch_oracle(b, rows=rows)
    got = to_np_f32(out)
    if rows is not None:
        got, ref = got[rows], ref[rows]
    vmax = float(b.value.float().abs().max())
    kmax = float(b.key.float().abs().max())
    assert vmax > 3 * vs and kmax > 3 * ks  # the draws reached the scales
    atol = 2e-3 * max(1.0, vmax / 4) * (max(1.0, kmax / 4) if ks > 1 else 1.0)
    assert_close(got, ref, atol=atol)


BIG_K = [
    # name, seq_lens, q_lens, Hq, Hkv
    ("fresh200_8x8", [200], [200], 8, 8),
    ("chunk20_ctx2k_48x8", [2000 + 20], [20], 48, 8),
    ("mixed_decode_48x8", [3000, 900 + 150, 500], [1, 150, 1], 48, 8),
]


@pytest.mark.parametrize("case", BIG_K, ids=[c[0] for c in BIG_K])
def test_keys_near_fp16_limit(case):
    """Keys up to 60000 at a softmax scale whose c = scale * log2 e has a
    mantissa near 1 (0.0858: c = 0.99 * 2^-3).  The prefill kernel's K^ =
    fp16(q * d_k * kmul) must stay finite wherever the decode kernel's
    fp16(q * d_k) is, so kmul is kept in [0.5, 1).  Queries at 5e-4 x N(0, 1)
    keep the scores at a few units; their error, and the bound, scale with
    the score magnitude."""
    need_gpu()
    name, sls, qls, Hq, Hkv = case
    announce(f"big keys {name}")
    b = W.build_batch(sls, qls, Hq, Hkv, seed=sum(map(ord, name)), write_cache=False)
    b.key = (b.key.float() * 12000).clamp(-60000, 60000).to(b.key.dtype)
    b.query = (b.query.float() * 5e-4).to(b.query.dtype)
    b.scale = 0.0858
    kp, vp = b.planes()
    import gfx906_fa
    gfx906_fa.reshape_and_cache_q8_kv(b.key, b.value, b.slot_mapping, kp, vp)
    out = W.attention(b, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert float(b.key.float().abs().max()) > 40000
    # score magnitude: |q| |k| scale over the head dim
    s_std = float(b.query.float().std() * b.key.float().std()) * 128 ** 0.5 * b.scale
    assert 1.0 < s_std < 20.0, s_std
    assert_close(to_np_f32(out), batch_oracle(b), atol=2e-3 * max(1.0, s_std))
