"""CPU: the committed golden fixtures agree with the oracle and the C
restatement (a fixture that drifts from the oracle, or an oracle change that
moves the fixtures, fails here)."""
import math
import os

import numpy as np

from oracle import c_oracle as C
from oracle import q8_oracle as O

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def test_cfg1_fixture_consistent():
    g = np.load(os.path.join(HERE, "q8_cfg1.npz"))
    k, v, q = g["key"], g["value"], g["query"]
    assert k.shape == (1024, 1, 128) and q.shape == (1, 8, 128)
    assert np.array_equal(C.quantize_rows(k), g["k_rows"])
    assert np.array_equal(C.quantize_rows(v), g["v_rows"])
    ka, va = O.planar_to_aos(g["cache"])
    bs = int(g["block_size"])
    slots = g["slot_mapping"]
    assert np.array_equal(ka[slots // bs, slots % bs], g["k_rows"])
    assert np.array_equal(va[slots // bs, slots % bs], g["v_rows"])
    kh, vh = O.planar_dequant(g["cache"])
    out = O.paged_attention_ref(q.astype(np.float32), kh, vh, g["block_table"], g["seq_lens"],
                                g["query_start_loc"], 1.0 / math.sqrt(128))
    # float64 throughout: equal up to the summation order of the products
    np.testing.assert_allclose(out, g["out"], rtol=0, atol=1e-12)
    # sanity: the output is a convex combination of V rows
    assert np.all(np.abs(out) <= np.abs(vh).max() + 1e-9)


def test_edge_fixture_consistent():
    g = np.load(os.path.join(HERE, "q8_edge.npz"))
    assert np.array_equal(O.quantize_q8_0_rows(g["f16"]), g["f16_rows"])
    assert np.array_equal(C.quantize_rows(g["f16"]), g["f16_rows"])
    assert np.array_equal(O.quantize_q8_0_rows(g["bf16_bits"]), g["bf16_rows"])
    assert np.array_equal(C.quantize_rows(g["bf16_bits"]), g["bf16_rows"])
    # row 0: ties -> even
    assert g["f16_rows"][0, 2:10].view(np.int8).tolist() == [127, -127, 0, 2, 2, 0, -2, -2]
