"""CPU: pin the Q8_0 oracle (quantizer, AoS format, dequant).

The oracle restates extension/gfx906_fa_quant.cu:45-85.  These checks do not
retype its formula: they compare it with an independent C restatement, with
the reference test's own float64 oracle (tests/test_quant.py:29-52, within
that test's tolerance, tests/test_quant.py:72-73), and with answers fixed by
arithmetic (ties, zero blocks, exact integer blocks, error bounds)."""
import numpy as np
import pytest

from oracle import c_oracle as C
from oracle import q8_oracle as O


def _inputs(rng, dt, shape, scale=1.0):
    x = (rng.standard_normal(shape) * scale).astype(np.float32)
    if dt == "f16":
        return x.astype(np.float16)
    if dt == "bf16":
        return O.f32_to_bf16_bits(x)
    return x


@pytest.mark.parametrize("dt", ["f16", "bf16", "f32"])
@pytest.mark.parametrize("scale", [1e-3, 0.5, 1.0, 37.0])
def test_numpy_matches_c_restatement(dt, scale):
    rng = np.random.default_rng(7)
    x = _inputs(rng, dt, (513, 128), scale)
    assert np.array_equal(O.quantize_q8_0_rows(x), C.quantize_rows(x))


@pytest.mark.parametrize("dt", ["f16", "bf16"])
def test_within_reference_f64_oracle_tolerance(dt):
    rng = np.random.default_rng(42)
    for shape in [(1, 32), (4, 128), (2, 8, 128), (1, 4, 64, 128)]:
        x = _inputs(rng, dt, shape, 0.5)
        ours = O.quantize_q8_0_rows(x).astype(int)
        ref = O.ref_quantize_f64(x).astype(int)
        diff = np.abs(ours - ref)
        assert diff.max() <= 1
        assert (diff > 0).mean() < 0.01


def test_known_answers_ties_and_extremes():
    # amax = 127 -> d = 1 exactly, id = 1: q = rint-half-even(x)
    blk = np.zeros(32, np.float32)
    blk[:8] = [127.0, -127.0, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5]
    q, d = O.quantize_q8_0_blocks(blk.astype(np.float16)[None])
    assert d[0, 0] == np.float16(1.0)
    assert q[0, :8].tolist() == [127, -127, 0, 2, 2, 0, -2, -2]
    # a round-half-away-from-zero quantizer would give 1, 3, 3, ... here
    rows = O.pack_q8_0_rows(q, d)
    assert rows[0, :2].tolist() == [0x00, 0x3C]  # fp16 1.0 little-endian


def test_zero_block_and_signed_zero():
    x = np.zeros((1, 64), np.float16)
    x[0, 33] = -0.0
    rows = O.quantize_q8_0_rows(x)
    assert not rows.any()


def test_amax_maps_to_127():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((200, 32)).astype(np.float16)
    q, _ = O.quantize_q8_0_blocks(x)
    a = np.abs(x.astype(np.float32))
    idx = np.argmax(a, axis=1)
    assert np.all(np.abs(q[np.arange(200), idx]) == 127)
    assert np.all(q[np.arange(200), idx] * np.sign(x[np.arange(200), idx]) > 0)


def test_integer_blocks_roundtrip_exactly():
    # blocks whose amax is 127 * 2^k with integer multiples survive exactly
    rng = np.random.default_rng(5)
    ints = rng.integers(-127, 128, size=(64, 32)).astype(np.float32)
    ints[:, 0] = 127.0
    for k in (-6, 0, 3):
        x = (ints * np.float32(2.0 ** k)).astype(np.float16)
        deq = O.dequantize_q8_0_rows(O.quantize_q8_0_rows(x), 32)
        assert np.array_equal(deq, x.astype(np.float32))


@pytest.mark.parametrize("dt", ["f16", "bf16"])
def test_dequant_error_bound(dt):
    rng = np.random.default_rng(11)
    x = _inputs(rng, dt, (1000, 128), 2.0)
    xf = O._to_f32(x)
    q, d = O.quantize_q8_0_blocks(x)
    deq = O.dequantize_blocks(q, d)
    dd = np.repeat(d.astype(np.float32), 32, axis=-1)
    # |x - q*fp16(d)| <= fp16(d)/2 + 127*|fp16(d) - d32| (scale rounding) + tiny
    d32 = np.repeat((np.max(np.abs(xf.reshape(1000, 4, 32)), -1) / np.float32(127)), 32, -1)
    bound = dd / 2 + 127.5 * np.abs(dd - d32) + 1e-7
    assert np.all(np.abs(deq - xf) <= bound)


def test_tiny_and_huge_blocks_match_c():
    # bf16 extremes: subnormal fp16 scales, fp16 overflow of the scale, and
    # blocks whose 1/d overflows (saturating int conversion)
    vals = np.array([1e-30, 3e-39, 1e-5, 7e4, 3e38], np.float32)
    blocks = []
    for v in vals:  # finite inputs only: NaN / inf are outside the contract
        blocks.append((np.linspace(-1.0, 1.0, 32) * v).astype(np.float32))
    x = O.f32_to_bf16_bits(np.stack(blocks))
    assert np.array_equal(O.quantize_q8_0_rows(x), C.quantize_rows(x))
    xh = np.stack([np.linspace(-1.0, 1.0, 32) * v for v in (6e-8, 1e-6, 6e4)]).astype(np.float16)
    assert np.array_equal(O.quantize_q8_0_rows(xh), C.quantize_rows(xh))


def test_aos_layout_offsets():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((3, 128)).astype(np.float16)
    rows = O.quantize_q8_0_rows(x)
    assert rows.shape == (3, 136)
    q, d = O.quantize_q8_0_blocks(x)
    for b in range(4):
        assert np.array_equal(rows[:, 34 * b:34 * b + 2].copy().view("<f2")[:, 0], d[:, b])
        assert np.array_equal(rows[:, 34 * b + 2:34 * b + 34].view(np.int8), q[:, 32 * b:32 * b + 32])
    q2, d2 = O.unpack_q8_0_rows(rows, 128)
    assert np.array_equal(q2, q) and np.array_equal(d2, d)
