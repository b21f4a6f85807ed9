"""CPU: pins of the rotary-embedding restatement (``oracle.q8_oracle.rope_ref``).

The arithmetic is vLLM's (its rotary embedding; vLLM is absent here), which
the reference backend would reach through fused_rope_kvcache_supported
(extension/gfx906_fa_backend.py:444-445).  Pins: an independent torch CPU
restatement of vLLM's native form with 16-bit tensor ops (bit for bit), the
float64 complex product for the pairing and signs, identity at angle 0,
pairwise norms, unchanged out-of-range rows, and planted mistakes that the
complex check must reject."""
import numpy as np
import pytest
import torch

from oracle import q8_oracle as O

TD = {"f16": torch.float16, "bf16": torch.bfloat16}
EPS = {"f16": 2.0 ** -10, "bf16": 2.0 ** -7}


def _inputs(dt, T=37, H=3, rot=128, P=4096, seed=0, cs_dtype="f32"):
    rng = np.random.default_rng(seed)
    x32 = (rng.standard_normal((T, H, 128)) * 2.0).astype(np.float32)
    x = O.f32_to_bf16_bits(x32) if dt == "bf16" else x32.astype(np.float16)
    cs = O.rope_cos_sin_cache(P, rot)
    if cs_dtype == "model":
        cs = O.f32_to_bf16_bits(cs) if dt == "bf16" else cs.astype(np.float16)
    pos = rng.integers(0, P, T).astype(np.int64)
    return x, pos, cs


def _to_torch(a, dt):
    a = np.asarray(a)
    if a.dtype == np.uint16:
        return torch.from_numpy(a.view(np.int16).copy()).view(torch.bfloat16)
    return torch.from_numpy(a.copy())


def _from_torch(t):
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def _torch_native_rope(x, positions, cos_sin, rot, neox):
    """vLLM's native form (RotaryEmbedding.forward_native) with torch ops."""
    cs = cos_sin[positions]
    cos, sin = cs.chunk(2, dim=-1)
    cos = cos.unsqueeze(-2).to(x.dtype)
    sin = sin.unsqueeze(-2).to(x.dtype)
    xr, xp = x[..., :rot], x[..., rot:]
    if neox:
        x1, x2 = torch.chunk(xr, 2, dim=-1)
    else:
        x1, x2 = xr[..., ::2], xr[..., 1::2]
    o1 = x1 * cos - x2 * sin
    o2 = x2 * cos + x1 * sin
    if neox:
        o = torch.cat((o1, o2), dim=-1)
    else:
        o = torch.stack((o1, o2), dim=-1).flatten(-2)
    return torch.cat((o, xp), dim=-1)


@pytest.mark.parametrize("dt", ["f16", "bf16"])
@pytest.mark.parametrize("neox", [True, False])
@pytest.mark.parametrize("rot", [128, 64])
@pytest.mark.parametrize("cs_dtype", ["f32", "model"])
def test_rope_matches_torch_native_form(dt, neox, rot, cs_dtype):
    x, pos, cs = _inputs(dt, rot=rot, cs_dtype=cs_dtype, seed=rot + neox)
    got = O.rope_ref(x, pos, cs, rot, neox)
    ref = _torch_native_rope(_to_torch(x, dt), torch.from_numpy(pos), _to_torch(cs, dt), rot, neox)
    assert np.array_equal(got, _from_torch(ref))


def _complex_ok(out, x, pos, cs, rot, neox, dt):
    """(x1 + i x2)(cos + i sin) in float64 against the output pairs, within a
    few roundings of the dtype."""
    xf = O._to_f32(x).astype(np.float64)
    of = O._to_f32(out).astype(np.float64)
    half = rot // 2
    c = O._round_model(O._to_f32(cs)[pos, :half], dt == "bf16").astype(np.float64)[:, None]
    s = O._round_model(O._to_f32(cs)[pos, half:rot], dt == "bf16").astype(np.float64)[:, None]
    sl1, sl2 = (slice(0, half), slice(half, rot)) if neox else (slice(0, rot, 2), slice(1, rot, 2))
    z = (xf[..., sl1] + 1j * xf[..., sl2]) * (c + 1j * s)
    tol = 4 * EPS[dt] * np.maximum(np.abs(xf[..., sl1]), np.abs(xf[..., sl2])) + 1e-30
    return (np.all(np.abs(of[..., sl1] - z.real) <= tol) and np.all(np.abs(of[..., sl2] - z.imag) <= tol)
            and np.array_equal(of[..., rot:], xf[..., rot:]))


@pytest.mark.parametrize("dt", ["f16", "bf16"])
@pytest.mark.parametrize("neox", [True, False])
def test_rope_is_the_complex_rotation(dt, neox):
    x, pos, cs = _inputs(dt, seed=3)
    assert _complex_ok(O.rope_ref(x, pos, cs, 128, neox), x, pos, cs, 128, neox, dt)
    x, pos, cs = _inputs(dt, rot=64, seed=4)
    assert _complex_ok(O.rope_ref(x, pos, cs, 64, neox), x, pos, cs, 64, neox, dt)


def test_rope_planted_mistakes_are_rejected():
    """The complex check fails for a swapped pairing, a flipped sign and a
    cos/sin swap, so it pins the restatement's conventions."""
    x, pos, cs = _inputs("f16", seed=5)
    good = O.rope_ref(x, pos, cs, 128, True)
    assert _complex_ok(good, x, pos, cs, 128, True, "f16")
    assert not _complex_ok(O.rope_ref(x, pos, cs, 128, False), x, pos, cs, 128, True, "f16")
    flipped = cs.copy()
    flipped[:, 64:] = -flipped[:, 64:]
    assert not _complex_ok(O.rope_ref(x, pos, flipped, 128, True), x, pos, cs, 128, True, "f16")
    swapped = np.concatenate([cs[:, 64:], cs[:, :64]], axis=1)
    assert not _complex_ok(O.rope_ref(x, pos, swapped, 128, True), x, pos, cs, 128, True, "f16")


@pytest.mark.parametrize("dt", ["f16", "bf16"])
@pytest.mark.parametrize("neox", [True, False])
def test_rope_signed_zeros_match_torch(dt, neox):
    """Zeros of both signs at angle 0 and elsewhere: IEEE zero signs of the
    products and differences agree with torch's 16-bit ops."""
    x, pos, cs = _inputs(dt, T=16, seed=8)
    xf = O._to_f32(x).copy()
    xf[:, :, ::3] = -0.0
    xf[:, :, 1::5] = 0.0
    x = O.f32_to_bf16_bits(xf) if dt == "bf16" else xf.astype(np.float16)
    pos[:8] = 0
    got = O.rope_ref(x, pos, cs, 128, neox)
    ref = _torch_native_rope(_to_torch(x, dt), torch.from_numpy(pos), _to_torch(cs, dt), 128, neox)
    assert np.array_equal(got.view(np.uint16), _from_torch(ref).view(np.uint16))


@pytest.mark.parametrize("dt", ["f16", "bf16"])
def test_rope_identity_norms_and_out_of_range(dt):
    x, pos, cs = _inputs(dt, seed=6)
    pos0 = np.zeros_like(pos)                      # angle 0: cos 1, sin 0 exactly
    assert np.array_equal(O.rope_ref(x, pos0, cs, 128, True), x)
    assert np.array_equal(O.rope_ref(x, pos0, cs, 128, False), x)
    out = O._to_f32(O.rope_ref(x, pos, cs, 128, True)).astype(np.float64)
    xf = O._to_f32(x).astype(np.float64)
    n0 = xf[..., :64] ** 2 + xf[..., 64:] ** 2
    n1 = out[..., :64] ** 2 + out[..., 64:] ** 2
    assert np.allclose(n1, n0, rtol=16 * EPS[dt], atol=1e-6)
    bad = pos.copy()
    bad[[0, 5]] = [-1, cs.shape[0]]
    got = O.rope_ref(x, bad, cs, 128, True)
    assert np.array_equal(got[[0, 5]], x[[0, 5]])
    assert np.array_equal(got[1:5], O.rope_ref(x[1:5], pos[1:5], cs, 128, True))
