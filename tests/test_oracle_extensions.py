"""Pins the oracle's restatement of the two benchmark extensions that the
reference does not have: per-head-scaled fp8 keys (k_head_scale,
encode_fp8_scaled, the far_k_scale argument of the attention oracles) and
the top-K spike selection (spike_topk, the far scores of attend_kernel).

Each check is an independent route to the same answer: exact power-of-two
scalings (where dividing is exponent arithmetic), the unscaled encoder on
every fp16 pattern, an E4M3 error bound, Python's own sort over (score,
index) pairs, and an fp64 brute-force softmax."""

import numpy as np
import pytest

import oracle

ALL_FP16 = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16)


def _finite(x):
    return x[np.isfinite(x.astype(np.float32))]


def test_scale_one_is_the_unscaled_encoder_on_every_pattern():
    x = ALL_FP16.reshape(1, 1, 512, 128)
    got = oracle.encode_fp8_scaled(x, np.ones((1, 1), np.float32))
    assert np.array_equal(got, oracle.encode_fp8(x))


@pytest.mark.parametrize("k", [-3, -1, 2, 5])
def test_power_of_two_scale_is_exponent_arithmetic(k):
    # dividing by 2^k is exact in fp32; the fp16 rounding then only bites
    # below the fp16 normal range or above 65504, which are excluded
    x = _finite(ALL_FP16)
    y = np.ldexp(x.astype(np.float64), -k)
    keep = (np.abs(y) >= 2.0 ** -14) & (np.abs(y) <= 60000) | (x == 0)
    x = x[keep]
    x = x[: (x.size // 64) * 64].reshape(1, 1, -1, 64)
    scale = np.full((1, 1), 2.0 ** k, np.float32)
    got = oracle.encode_fp8_scaled(x, scale)
    want = oracle.encode_fp8(np.ldexp(x.astype(np.float64), -k).astype(np.float16))
    assert np.array_equal(got, want)


def test_head_amax_encodes_to_0x77_and_codes_stay_finite():
    rng = np.random.default_rng(3)
    keys = (rng.standard_normal((2, 3, 200, 64)) * rng.choice([0.01, 1, 40, 900], (2, 3, 1, 1))).astype(np.float16)
    s = oracle.k_head_scale(keys)
    codes = oracle.encode_fp8_scaled(keys, s)
    for b in range(2):
        for h in range(3):
            i = np.unravel_index(np.argmax(np.abs(keys[b, h].astype(np.float32))), keys[b, h].shape)
            assert codes[b, h][i] & 0x7F == 0x77
            assert s[b, h] == np.float32(np.abs(keys[b, h].astype(np.float32)).max()) / np.float32(240)
    assert (codes & 0x7F).max() <= 0x77  # never the saturation or NaN codes


def test_scaled_decode_error_bound():
    # E4M3 keeps 3 mantissa bits: |decode(code)*scale - x| <= 2^-4 |x| (+ the
    # fp16 rounding of x/scale) wherever x/scale is in E4M3's normal range
    rng = np.random.default_rng(5)
    keys = (rng.standard_normal((1, 4, 300, 128)) * np.array([1e-3, 1, 50, 3000])[None, :, None, None]).astype(np.float16)
    s = oracle.k_head_scale(keys)
    dec = oracle.decode_fp8(oracle.encode_fp8_scaled(keys, s)).astype(np.float64) * s[..., None, None]
    x = keys.astype(np.float64)
    normal = np.abs(x) / s[..., None, None] >= 2.0 ** -6
    err = np.abs(dec - x)[normal] / np.abs(x)[normal]
    assert err.max() <= 2.0 ** -4 * (1 + 2.0 ** -10) + 2.0 ** -11
    # the unscaled encoder flushes keys below 2^-6 to zero; scaled they survive
    small = keys[0, 0]
    assert np.count_nonzero(oracle.encode_fp8(small) & 0x7F) < 0.5 * small.size
    assert np.count_nonzero(oracle.encode_fp8_scaled(keys, s)[0, 0] & 0x7F) > 0.95 * small.size


def test_zero_heads_and_non_finite_keys():
    keys = np.zeros((1, 2, 64, 64), np.float16)
    keys[0, 1, 3, 5] = np.inf
    keys[0, 1, 4, 6] = 2.0
    s = oracle.k_head_scale(keys)
    assert s[0, 0] == 1.0 and s[0, 1] == np.float32(2.0) / np.float32(240)
    c = oracle.encode_fp8_scaled(keys, s)
    assert c[0, 1, 3, 5] == 0x7E and c[0, 1, 4, 6] == 0x77 and not c[0, 0].any()


def test_scale_448_would_saturate_the_top_of_the_range():
    # why the scale maps amax to 240: the Metal encoder sends every input
    # from 240 (after rounding) up to the saturation code
    x = np.array([239.0, 240.0, 247.9, 248.0, 300.0, 447.0], np.float16)
    assert list(oracle.encode_fp8(x)) == [0x77, 0x77, 0x77, 0x7E, 0x7E, 0x7E]


def _tiny(seed, B=1, Hq=4, Hkv=2, D=64, Npad=64, F=150, n_dec=3, scale=None):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((B, Hq, D)).astype(np.float16)
    nk = rng.standard_normal((B, Hkv, Npad, D)).astype(np.float16)
    nv = rng.standard_normal((B, Hkv, Npad, D)).astype(np.float16)
    fk_src = (rng.standard_normal((B, Hkv, F, D)) * 3).astype(np.float16)
    fv_src = rng.standard_normal((B, Hkv, F, D)).astype(np.float16)
    ks = oracle.k_head_scale(fk_src) if scale is None else scale
    fk = oracle.encode_fp8_scaled(fk_src, ks)
    fv, fs, fz = oracle.quant_int4(fv_src)
    dk = rng.standard_normal((B, Hkv, n_dec, D)).astype(np.float16)
    dv = rng.standard_normal((B, Hkv, n_dec, D)).astype(np.float16)
    valid = np.full(Hkv, Npad - 5, np.int32)
    return q, nk, nv, valid, fk, fv, fs, fz, dk, dv, ks


def test_kernel_oracle_scale_equals_prescaled_fp16_keys():
    # with power-of-two scales decode(code) * scale is an exact fp16 value,
    # so passing the scale must equal passing those fp16 keys
    ks = np.array([[0.25, 8.0]], np.float32)
    q, nk, nv, valid, fk, fv, fs, fz, dk, dv, _ = _tiny(1, scale=ks)
    k16 = (oracle.decode_fp8(fk).astype(np.float32) * ks[..., None, None]).astype(np.float16)
    a = oracle.attend_kernel(q, nk, nv, valid, fk, fv, fs, fz, dk, dv, far_k_scale=ks, return_far_scores=True)
    b = oracle.attend_kernel(q, nk, nv, valid, None, fv, fs, fz, dk, dv, far_k_f16=k16, return_far_scores=True)
    for x, y in zip(a, b):
        assert np.array_equal(x, y)


def test_formulation_with_scale_is_brute_force_softmax():
    q, nk, nv, valid, fk, fv, fs, fz, dk, dv, ks = _tiny(2)
    got = oracle.attend_formulation(q, nk, nv, valid, fk, fv, fs, fz, dk, dv, far_k_scale=ks)
    B, Hq, D = q.shape
    Hkv = nk.shape[1]
    G = Hq // Hkv
    far_k = oracle.decode_fp8(fk).astype(np.float32) * ks[..., None, None]
    far_v = np.stack([np.stack([(((fv[..., j // 2] >> (4 * (j % 2))) & 15).astype(np.float32)
                                 * fs.astype(np.float32)).astype(np.float16).astype(np.float32)
                                for j in range(D)], -1)], 0)[0]
    far_v = (far_v + fz.astype(np.float32)[..., None]).astype(np.float16).astype(np.float64)
    for b in range(B):
        for h in range(Hq):
            kv = h // G
            n = int(valid.max())
            K = np.concatenate([nk[b, kv, :n].astype(np.float64), dk[b, kv].astype(np.float64),
                                far_k[b, kv].astype(np.float64)])
            V = np.concatenate([nv[b, kv, :n].astype(np.float64), dv[b, kv].astype(np.float64), far_v[b, kv]])
            s = K @ q[b, h].astype(np.float64) / np.sqrt(D)
            w = np.exp(s - s.max())
            assert np.allclose(got[b, h], w @ V / w.sum(), rtol=0, atol=1e-9)


def _brute_topk(scores, thr, K):
    """Python's sort over (-score, index): descending score, then index."""
    order = [i for _, i in sorted((-float(x), i) for i, x in enumerate(scores))]
    n = min(K, sum(1 for x in scores if x > thr))
    tok = [-1] * K
    tok[:n] = order[:n]
    if order:
        tok[0] = order[0]
    return n, tok


@pytest.mark.parametrize("K", [1, 2, 7, 32])
def test_spike_topk_matches_python_sort(K):
    rng = np.random.default_rng(K)
    B, Hq, F = 2, 5, 300
    sc = rng.standard_normal((B, Hq, F)).round(1)  # many exact ties
    sc[0, 1] = 0.0                                  # all tied
    sc[1, 2, 40:90] += 9.0                          # a block of spikes
    mn = rng.standard_normal((B, Hq)) - 1.0
    margin = 2.0
    cnt, tok = oracle.spike_topk(sc, mn, margin, K)
    for b in range(B):
        for h in range(Hq):
            n, t = _brute_topk(sc[b, h], mn[b, h] + margin, K)
            assert cnt[b, h] == n and list(tok[b, h]) == t, (b, h)


def test_spike_topk_k1_is_the_kernel_flag_and_token():
    q, nk, nv, valid, fk, fv, fs, fz, dk, dv, ks = _tiny(4, F=400)
    # plant spikes: far keys aligned with a query
    out, flags, tokens, mf, mn, fsc = oracle.attend_kernel(q, nk, nv, valid, fk, fv, fs, fz, dk, dv, spike_margin=1.0,
                                                           far_k_scale=ks, return_far_scores=True)
    assert np.array_equal(fsc.max(-1), mf)
    cnt, tok = oracle.spike_topk(fsc, mn, 1.0, 1)
    assert np.array_equal(cnt, flags) and np.array_equal(tok[..., 0], tokens)
    cnt8, tok8 = oracle.spike_topk(fsc, mn, 1.0, 8)
    assert np.array_equal(tok8[..., 0], tokens)
    assert np.array_equal(cnt8 > 0, flags > 0)


def test_spike_topk_empty_far_tier():
    cnt, tok = oracle.spike_topk(np.zeros((1, 2, 0)), np.zeros((1, 2)), 0.5, 4)
    assert not cnt.any() and (tok == -1).all()
