"""Pins the oracle's fp8 / INT4 codecs (CPU only).

Each check is independent of the oracle's bit manipulation: value-semantics
restatements in float64 numpy, torch's own float8_e4m3fn conversions, and
invariants / crafted cases of the quantiser.
"""

import numpy as np
import pytest
import torch

ALL16 = np.arange(65536, dtype=np.uint16)


def _grid_round(a, python=False):
    """Value semantics of the reference E4M3 encoders on |x| (float64).

    Metal (foveated_compress.metal:39-66): |x| < 2^-6 -> 0, |x| >= 256 -> 448,
    else round-half-even to the E4M3 grid, and a result >= 256 -> 448.
    Python (mlx_foveated.py:528-566): round first on the fp16 exponent's
    binade, results < 2^-6 -> 0, results >= 256 (or inf/nan) -> 224."""
    out = np.zeros_like(a)
    with np.errstate(divide="ignore", invalid="ignore"):
        E = np.floor(np.log2(np.where(a > 0, a, 1.0)))
    q = np.exp2(E - 3)
    with np.errstate(invalid="ignore"):
        y = np.round(a / q) * q  # numpy rounds half to even
    if not python:
        mid = (a >= 2.0 ** -6) & (a < 256.0)
        out[mid] = y[mid]
        out[(a >= 256.0) | (mid & (y >= 256.0))] = 448.0
    else:
        ok = (a >= 2.0 ** -7) & np.isfinite(a)
        res = np.where(ok, y, 0.0)
        res = np.where(res < 2.0 ** -6, 0.0, res)
        res = np.where((res >= 256.0) | ~np.isfinite(a), 224.0, res)
        out = res
    return out


def _decode_value(codes):
    c = codes.astype(np.int64)
    s = np.where(c >> 7, -1.0, 1.0)
    e = (c >> 3) & 15
    m = c & 7
    v = np.where(e == 0, 0.0, np.exp2(e - 7.0) * (1 + m / 8.0))
    return s * v


@pytest.mark.parametrize("python", [False, True])
def test_fp8_encoder_value_semantics_exhaustive(orc, python):
    codes = orc.encode_fp8(ALL16, python_semantics=python)
    x = ALL16.view(np.float16).astype(np.float64)
    a = np.abs(x)
    a = np.where(np.isnan(x), np.inf, a)
    expect = _grid_round(a, python=python)
    got = np.abs(_decode_value(codes))
    assert np.array_equal(got, expect)
    # sign is carried through for every pattern (including zeros)
    assert np.array_equal(codes >> 7, (ALL16 >> 15).astype(np.uint8))


def test_fp8_encoder_matches_torch_rne_on_normal_range(orc):
    x = ALL16.view(np.float16)
    xf = x.astype(np.float32)
    sel = np.isfinite(xf) & (np.abs(xf) >= 2.0 ** -6) & (np.abs(xf) < 240.0)
    t = torch.from_numpy(xf[sel]).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    ours = orc.encode_fp8(x[sel])
    # torch keeps -0/+0 sign and is RNE: identical codes on the normal range
    assert np.array_equal(ours, t)


def test_fp8_encoder_divergence_between_reference_encoders(orc):
    metal = orc.encode_fp8(ALL16)
    py = orc.encode_fp8(ALL16, python_semantics=True)
    diff = metal != py
    # 18,688 fp16 patterns disagree (an exhaustive count); all sit in the underflow
    # rounding band or at/above the overflow threshold
    assert int(diff.sum()) == 18688
    a = np.abs(ALL16[diff].view(np.float16).astype(np.float64))
    a = np.where(np.isnan(a), np.inf, a)
    assert np.all(((a >= 0.0151367) & (a < 2.0 ** -6)) | (a >= 240.0))


def test_fp8_decode_lut_closed_form_and_torch(orc):
    codes = np.arange(256, dtype=np.uint8)
    ours = orc.decode_fp8(codes).astype(np.float64)
    assert np.array_equal(np.abs(ours), np.abs(_decode_value(codes)))
    e = (codes >> 3) & 15
    normal = (e > 0) & ((codes & 0x7F) != 0x7F)
    t = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy().astype(np.float64)
    assert np.array_equal(ours[normal], t[normal])
    # code 0x7F decodes to 480 in the reference LUT (E4M3FN NaN slot)
    assert ours[0x7F] == 480.0 and ours[0xFF] == -480.0


def test_fp8_reachable_code_set(orc):
    codes = np.unique(orc.encode_fp8(ALL16))
    assert codes.size == 228
    e = (codes >> 3) & 15
    m = codes & 7
    assert not np.any((e == 0) & (m != 0))  # no subnormal codes
    assert not np.any((codes & 0x7F) == 0x7F)  # no NaN slot
    assert codes.max() == 0xFE and (codes & 0x7F).max() == 0x7E


def test_fp8_roundtrip_quality(orc):
    rng = np.random.default_rng(0)
    x = rng.standard_normal((2, 32, 64)).astype(np.float16)
    y = orc.decode_fp8(orc.encode_fp8(x)).astype(np.float64)
    assert orc.cosine(x, y) > 0.95  # tests/test_mlx_foveated.py:133-144
    z = np.zeros(32, np.float16)
    assert np.all(orc.decode_fp8(orc.encode_fp8(z)) == 0)


# ---------------------------------------------------------------------------
# INT4 per-token
# ---------------------------------------------------------------------------

def _unpack(packed):
    return np.stack([packed & 15, packed >> 4], -1).reshape(packed.shape[:-1] + (-1,))


@pytest.mark.parametrize("D", [64, 128])
def test_int4_invariants(orc, D):
    rng = np.random.default_rng(D)
    x = (rng.standard_normal((3, 50, D)) * rng.uniform(0.1, 8, (3, 50, 1))).astype(np.float16)
    packed, sc, zr = orc.quant_int4(x)
    c = _unpack(packed)
    assert c.shape == x.shape and c.max() <= 15
    xf = x.astype(np.float32)
    mn, mx = xf.min(-1), xf.max(-1)
    s32 = np.maximum((mx - mn) / np.float32(15), np.float32(1e-8))
    # stored scale / zero are the fp16 roundings of the fp32 values
    assert np.array_equal(sc, s32.astype(np.float16))
    assert np.array_equal(zr, mn.astype(np.float16))
    # the row min codes to 0 and the row max to 15
    am = np.argmin(xf, -1)
    aM = np.argmax(xf, -1)
    assert np.all(np.take_along_axis(c, am[..., None], -1) == 0)
    assert np.all(np.take_along_axis(c, aM[..., None], -1) == 15)
    # reconstruction error within half a step of the fp32 scale
    rec = c * s32[..., None] + mn[..., None]
    assert np.all(np.abs(rec - xf) <= s32[..., None] * 0.5 * (1 + 1e-5) + 1e-6)


@pytest.mark.parametrize("D", [64, 128])
def test_int4_group32_invariants(orc, D):
    """Group-32 INT4: every 32-dim group has its own fp32 min / range; the
    packing keeps dim d in byte d/2 (even dim low nibble) across groups."""
    rng = np.random.default_rng(D + 5)
    ng = D // 32
    mult = (3.0 ** np.arange(ng)).repeat(32)  # groups of very different ranges
    x = (rng.standard_normal((4, 40, D)) * mult + rng.uniform(-2, 2, (4, 40, 1))).astype(np.float16)
    packed, sc, zr = orc.quant_int4_groups(x, 32)
    assert packed.shape == (4, 40, D // 2) and sc.shape == zr.shape == (4, 40, ng)
    c = _unpack(packed)
    xf = x.astype(np.float32).reshape(4, 40, ng, 32)
    cg = c.reshape(4, 40, ng, 32)
    mn, mx = xf.min(-1), xf.max(-1)
    s32 = np.maximum((mx - mn) / np.float32(15), np.float32(1e-8))
    assert np.array_equal(sc, s32.astype(np.float16)) and np.array_equal(zr, mn.astype(np.float16))
    assert np.all(np.take_along_axis(cg, np.argmin(xf, -1)[..., None], -1) == 0)
    assert np.all(np.take_along_axis(cg, np.argmax(xf, -1)[..., None], -1) == 15)
    rec = cg * s32[..., None] + mn[..., None]
    assert np.all(np.abs(rec - xf) <= s32[..., None] * 0.5 * (1 + 1e-5) + 1e-6)
    # a group equal to a whole per-token row of 32 dims codes identically
    p1, s1, z1 = orc.quant_int4(x[..., 32:64])
    assert np.array_equal(p1, packed[..., 16:32]) and np.array_equal(s1, sc[..., 1])


def test_int4_ties_and_constant_rows(orc):
    # min 0, max 15 -> scale exactly 1: 2.5 and 7.5 are exact ties
    row = np.zeros(64, np.float32)
    row[1] = 15.0
    row[2] = 2.5
    row[3] = 7.5
    row[4] = 0.5
    x = row.astype(np.float16)[None]
    c_metal = _unpack(orc.quant_int4(x)[0])[0]
    c_py = _unpack(orc.quant_int4(x, python_semantics=True)[0])[0]
    assert list(c_metal[:5]) == [0, 15, 3, 8, 1]  # half away from zero
    assert list(c_py[:5]) == [0, 15, 2, 8, 0]  # half to even
    # even dims go to the low nibble
    assert orc.quant_int4(x)[0][0, 0] == (0 | (15 << 4))
    # constant row: codes 0; Metal scale half(1e-8) == 0, Python scale 1
    k = np.full((1, 64), 3.0, np.float16)
    p, s, z = orc.quant_int4(k)
    assert np.all(p == 0) and s[0] == 0 and z[0] == np.float16(3.0)
    p, s, z = orc.quant_int4(k, python_semantics=True)
    assert np.all(p == 0) and s[0] == 1 and z[0] == np.float16(3.0)


def test_int4_roundtrip_quality(orc):
    rng = np.random.default_rng(3)
    x = rng.standard_normal((2, 32, 64)).astype(np.float16)
    p, s, z = orc.quant_int4(x)
    rec = orc.dequant_int4_fp32(p, s, z)
    assert orc.cosine(x, rec) > 0.90  # tests/test_mlx_foveated.py:185-206
