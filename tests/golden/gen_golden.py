"""Writes the committed golden fixtures from the CPU oracle.

    python tests/golden/gen_golden.py

q8_cfg1.npz - the benchmark's CPU configuration (cfg1): one sequence of 1024
  tokens, 8 query heads / 1 KV head, head_dim 128, block_size 16, randomly
  permuted block table, fp16 K/V/Q ~ N(0,1) from numpy seed 20261201, one
  decode token, scale 1/sqrt(128).  Holds the inputs, the planar Q8 cache
  bytes, the AoS Q8_0 rows of K and V, and the float64 attention output.
q8_edge.npz - quantizer known answers: tie rows, zero rows, tiny / huge
  blocks in fp16 and bf16 (bit patterns), with their AoS bytes.

The reference publishes no vectors for this path (its tests draw inputs on
the GPU); these fixtures pin this build's oracle, which is itself pinned by
the checks in tests/test_oracle_*.py.
"""
import math
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import q8_oracle as O  # noqa: E402

SEED = 20261201


def cfg1():
    rng = np.random.default_rng(SEED)
    L, Hq, Hkv, D, bs = 1024, 8, 1, 128, 16
    nb = L // bs + 4
    perm = rng.permutation(nb)[: L // bs].astype(np.int32)
    bt = perm[None, :]
    k = rng.standard_normal((L, Hkv, D)).astype(np.float16)
    v = rng.standard_normal((L, Hkv, D)).astype(np.float16)
    q = rng.standard_normal((1, Hq, D)).astype(np.float16)
    pos = np.arange(L)
    slots = bt[0, pos // bs].astype(np.int64) * bs + pos % bs
    cache = np.zeros(O.planar_cache_shape(nb, bs, Hkv), np.uint8)
    O.planar_cache_write(k, v, slots, cache)
    k_rows = O.quantize_q8_0_rows(k)
    v_rows = O.quantize_q8_0_rows(v)
    kh, vh = O.planar_dequant(cache)
    sl = np.array([L], np.int32)
    qsl = np.array([0, 1], np.int32)
    out = O.paged_attention_ref(q.astype(np.float32), kh, vh, bt, sl, qsl, 1.0 / math.sqrt(D))
    return dict(key=k, value=v, query=q, block_table=bt, slot_mapping=slots, seq_lens=sl,
                query_start_loc=qsl, num_blocks=np.int32(nb), block_size=np.int32(bs),
                cache=cache, k_rows=k_rows, v_rows=v_rows, out=out)


def edge():
    rows = []
    t = np.zeros(32, np.float32)
    t[:8] = [127, -127, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5]
    rows.append(t)
    rows.append(np.zeros(32, np.float32))
    for v in (6e-8, 1e-6, 1e-3, 1.0, 6e4):
        rows.append((np.linspace(-1.0, 1.0, 32) * v).astype(np.float32))
    f16 = np.stack(rows).astype(np.float16)
    bvals = [1e-30, 1e-5, 3.0, 7e4, 3e38]
    b16 = O.f32_to_bf16_bits(np.stack([(np.linspace(-1.0, 1.0, 32) * v).astype(np.float32)
                                       for v in bvals]))
    return dict(f16=f16, f16_rows=O.quantize_q8_0_rows(f16), bf16_bits=b16,
                bf16_rows=O.quantize_q8_0_rows(b16))


def main():
    np.savez_compressed(os.path.join(HERE, "q8_cfg1.npz"), **cfg1())
    np.savez_compressed(os.path.join(HERE, "q8_edge.npz"), **edge())
    print("wrote", sorted(f for f in os.listdir(HERE) if f.endswith(".npz")))


if __name__ == "__main__":
    main()
