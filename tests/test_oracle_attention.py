"""Pins the oracle's tier plan and attention restatements (CPU only)."""

import glob
import os

import numpy as np
import pytest

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


# ---------------------------------------------------------------------------
# tier boundaries / split plan: known answers
# ---------------------------------------------------------------------------

def test_tier_boundaries_known_answer_s1000(orc):
    # tests/test_mlx_foveated.py:235-249: S=1000 -> 100 near valid, 900 far, padded
    tb = orc.tier_boundaries(1000)
    assert tb["R_actual"] == 100 and tb["far_count"] == 900
    assert tb["N_near_padded"] == 150  # headroom max(int(100*0.5), 8)


@pytest.mark.parametrize("S,R,F,headroom,npad", [
    (512, 51, 461, 25, 76),          # config 1
    (4096, 409, 3687, 204, 613),     # config 2
    (8192, 819, 7373, 409, 1228),    # config 3, 8K
    (16384, 1638, 14746, 819, 2457), # config 3, 16K
    (32768, 3276, 29492, 1638, 4914),
    (65536, 6553, 58983, 3276, 9829),  # config 5
])
def test_tier_boundaries_config_table(orc, S, R, F, headroom, npad):
    tb = orc.tier_boundaries(S)
    assert (tb["R_actual"], tb["far_count"], tb["headroom"], tb["N_near_padded"]) == (R, F, headroom, npad)
    # partition covers every position exactly once (near sets + far range)
    near, far, _ = orc.tier_indices(S, 1, 1)
    n = near[0, 0][near[0, 0] >= 0]
    allpos = np.sort(np.concatenate([n, far[0, 0]]))
    assert np.array_equal(allpos, np.arange(S))


@pytest.mark.parametrize("S", [0, 1, 3, 4, 20, 36, 37, 40, 100])
def test_tier_boundaries_short_sequences(orc, S):
    tb = orc.tier_boundaries(S)
    near, far, _ = orc.tier_indices(S, 1, 1)
    n = near[0, 0][near[0, 0] >= 0]
    assert n.size == tb["R_actual"] and far.shape[-1] == tb["far_count"]
    assert np.array_equal(np.sort(np.concatenate([n, far[0, 0]])), np.arange(S))
    assert tb["far_count"] >= 0 and tb["N_near_padded"] >= tb["R_actual"] + 8


@pytest.mark.parametrize("s_total,plan", [
    (553, (256, 3, 4)), (4364, (512, 9, 16)), (17203, (1280, 14, 16)), (256, (256, 1, 1)),
    (4096, (256, 16, 16)), (4097, (512, 9, 16)),
])
def test_split_plan_known_answers(orc, s_total, plan):
    assert orc.split_plan(s_total) == plan


# ---------------------------------------------------------------------------
# legacy golden vectors (reference tests/fixtures/*.pt, converted to npz)
# ---------------------------------------------------------------------------

def _legacy_inputs(z):
    f = lambda a: a.astype(np.float32)
    pk = (f(z["periph_k"]) * f(z["pk_scale"])[:, :, None, :] + f(z["pk_zero"])[:, :, None, :]).astype(np.float16)
    pv = (f(z["periph_v"]) * f(z["pv_scale"]) + f(z["pv_zero"])).astype(np.float16)
    fk = (f(z["far_k"]) * f(z["fak_scale"])[:, :, None, :] + f(z["fak_zero"])[:, :, None, :]).astype(np.float16)
    near_k = np.concatenate([z["foveal_k"], pk], 2)
    near_v = np.concatenate([z["foveal_v"], pv], 2)
    H = near_k.shape[1]
    return dict(
        q=z["query"][:, :, 0], near_k=near_k, near_v=near_v,
        near_valid=np.full(H, near_k.shape[2], np.uint32),
        far_k=None, far_k_f16=fk, far_v=z["far_v"],
        far_vs=z["fav_scale"][..., 0], far_vz=z["fav_zero"][..., 0],
    )


LEGACY = sorted(glob.glob(os.path.join(GOLDEN, "legacy_*.npz")))


@pytest.mark.parametrize("path", LEGACY, ids=[os.path.basename(p) for p in LEGACY])
def test_kernel_oracle_reproduces_legacy_fixture(orc, path):
    z = np.load(path)
    inp = _legacy_inputs(z)
    margin = float(z["spike_margin"])
    out, flags, tokens, mf, mn = orc.attend_kernel(
        inp["q"], inp["near_k"], inp["near_v"], inp["near_valid"], inp["far_k"],
        inp["far_v"], inp["far_vs"], inp["far_vz"], spike_margin=margin,
        far_k_f16=inp["far_k_f16"])
    ref = z["ref_output"][:, :, 0].astype(np.float64)
    assert np.abs(out - ref).max() < 6e-5  # fp16 half-ulp of the stored outputs
    # legacy spikes are per KV head = the first q head of each GQA group
    B, Hq = flags.shape
    Hkv = inp["near_k"].shape[1]
    G = Hq // Hkv
    lf = flags[:, ::G].reshape(-1)
    assert np.array_equal(lf, z["ref_spike_flags"])
    lt = np.where(lf == 1, tokens[:, ::G].reshape(-1), 0)  # legacy writes 0 when no spike
    assert np.array_equal(lt, z["ref_spike_tokens"])


def test_spike_case_is_flagged(orc):
    z = np.load(os.path.join(GOLDEN, "legacy_spike_case.npz"))
    assert list(z["ref_spike_flags"]) == [1, 1] and list(z["ref_spike_tokens"]) == [3, 7]


# ---------------------------------------------------------------------------
# brute force on small random inputs
# ---------------------------------------------------------------------------

def make_case(rng, B=1, Hq=8, Hkv=2, D=64, S=200, n_dec=5, near_valid_delta=0, orc=None, v_group=0):
    keys = rng.standard_normal((B, Hkv, S, D)).astype(np.float16)
    vals = rng.standard_normal((B, Hkv, S, D)).astype(np.float16)
    if v_group:  # value groups of very different ranges: a group index mix-up shows
        vals = (vals * (4.0 ** np.arange(D // v_group)).repeat(v_group)).astype(np.float16)
    c = orc.compress_layer(keys, vals, v_group=v_group)
    nv = c["near_valid"].astype(np.uint32) + np.uint32(near_valid_delta)
    q = rng.standard_normal((B, Hq, D)).astype(np.float16)
    dk = rng.standard_normal((B, Hkv, n_dec, D)).astype(np.float16) if n_dec else None
    dv = rng.standard_normal((B, Hkv, n_dec, D)).astype(np.float16) if n_dec else None
    return c, q, nv, dk, dv


def brute_force(q, c, nv, dk, dv, fp16_v=False):
    """Naive fp64 softmax over [near(valid) | far | decode] per q head."""
    B, Hq, D = q.shape
    Hkv = c["near_k"].shape[1]
    G = Hq // Hkv
    fk = c["far_k"]
    lut = np.array([(0 if ((i >> 3) & 15) == 0 else (1 if i < 128 else -1) * 2.0 ** (((i >> 3) & 15) - 7) * (1 + (i & 7) / 8)) for i in range(256)])
    fkd = lut[fk]
    lo = (c["far_v"] & 15).astype(np.float64)
    hi = (c["far_v"] >> 4).astype(np.float64)
    codes = np.stack([lo, hi], -1).reshape(fk.shape)
    if c["far_v_scale"].ndim == 4:  # one scale / zero per D/ng-dim group
        g = fk.shape[-1] // c["far_v_scale"].shape[-1]
        s16, z16 = np.repeat(c["far_v_scale"], g, -1), np.repeat(c["far_v_zero"], g, -1)
    else:
        s16, z16 = c["far_v_scale"][..., None], c["far_v_zero"][..., None]
    s = s16.astype(np.float64)
    zz = z16.astype(np.float64)
    if fp16_v:
        fvd = ((codes.astype(np.float16) * s16) + z16).astype(np.float64)
    else:
        fvd = codes * s + zz
    out = np.zeros((B, Hq, D))
    for b in range(B):
        for h in range(Hq):
            kv = h // G
            n = int(nv[kv])
            K = [c["near_k"][b, kv, :n].astype(np.float64), fkd[b, kv]]
            V = [c["near_v"][b, kv, :n].astype(np.float64), fvd[b, kv]]
            if dk is not None:
                K.append(dk[b, kv].astype(np.float64))
                V.append(dv[b, kv].astype(np.float64))
            K = np.concatenate(K)
            V = np.concatenate(V)
            sc = K @ q[b, h].astype(np.float64) / np.sqrt(D)
            w = np.exp(sc - sc.max())
            out[b, h] = w @ V / w.sum()
    return out


@pytest.mark.parametrize("shape", [
    dict(B=1, Hq=8, Hkv=2, D=64, S=200, n_dec=5),
    dict(B=2, Hq=4, Hkv=4, D=128, S=300, n_dec=0),
    dict(B=1, Hq=14, Hkv=2, D=64, S=512, n_dec=16),
])
def test_kernel_oracle_brute_force(orc, shape):
    rng = np.random.default_rng(7)
    c, q, nv, dk, dv = make_case(rng, orc=orc, **shape)
    out, *_ = orc.attend_kernel(q, c["near_k"], c["near_v"], nv, c["far_k"], c["far_v"],
                                c["far_v_scale"], c["far_v_zero"], dk, dv, gate=False)
    bf = brute_force(q, c, nv, dk, dv)
    # q is pre-scaled in fp32 by the kernel: relative 2^-24 perturbation only
    assert np.abs(out - bf).max() < 1e-6
    outg, *_ = orc.attend_kernel(q, c["near_k"], c["near_v"], nv, c["far_k"], c["far_v"],
                                 c["far_v_scale"], c["far_v_zero"], dk, dv, gate=True)
    assert np.abs(outg - bf).max() < 1e-4  # gated tokens weigh < e^-16 each


@pytest.mark.parametrize("D", [64, 128])
def test_kernel_and_formulation_oracle_group32_brute_force(orc, D):
    """Group-32 V (one scale / zero per 32 dims): both C restatements against
    the naive softmax over numpy-dequantised values."""
    rng = np.random.default_rng(D + 1)
    c, q, nv, dk, dv = make_case(rng, orc=orc, B=2, Hq=8, Hkv=2, D=D, S=333, n_dec=6, v_group=32)
    assert c["far_v_scale"].shape == c["far_k"].shape[:3] + (D // 32,)
    bf = brute_force(q, c, nv, dk, dv)
    out, *_ = orc.attend_kernel(q, c["near_k"], c["near_v"], nv, c["far_k"], c["far_v"],
                                c["far_v_scale"], c["far_v_zero"], dk, dv, gate=False)
    scale = np.abs(bf).max()
    assert np.abs(out - bf).max() < 1e-6 * scale
    fo = orc.attend_formulation(q, c["near_k"], c["near_v"], nv, c["far_k"], c["far_v"],
                                c["far_v_scale"], c["far_v_zero"], dk, dv)
    bf16 = brute_force(q, c, nv, dk, dv, fp16_v=True)
    assert np.abs(fo - bf16).max() < 1e-9 * scale


def test_kernel_oracle_split_invariance(orc):
    rng = np.random.default_rng(11)
    c, q, nv, dk, dv = make_case(rng, orc=orc, B=1, Hq=8, Hkv=2, D=64, S=700, n_dec=9)
    s_total = c["near_k"].shape[2] + c["far_k"].shape[2] + 9
    outs = []
    for n in (1, 2, 4, 8, 16):
        ss = -(-s_total // n)
        o, fl, tk, mf, mn = orc.attend_kernel(q, c["near_k"], c["near_v"], nv, c["far_k"],
                                              c["far_v"], c["far_v_scale"], c["far_v_zero"],
                                              dk, dv, split_size=ss, num_splits=n, gate=False,
                                              spike_margin=0.0)
        outs.append((o, fl, tk, mf, mn))
    for o, fl, tk, mf, mn in outs[1:]:
        assert np.abs(o - outs[0][0]).max() < 1e-12
        assert np.array_equal(tk, outs[0][2]) and np.array_equal(fl, outs[0][1])


def test_kernel_oracle_spike_semantics_brute_force(orc):
    rng = np.random.default_rng(5)
    c, q, nv, dk, dv = make_case(rng, orc=orc, B=2, Hq=8, Hkv=2, D=64, S=400, n_dec=4)
    o, fl, tk, mf, mn = orc.attend_kernel(q, c["near_k"], c["near_v"], nv, c["far_k"], c["far_v"],
                                          c["far_v_scale"], c["far_v_zero"], dk, dv,
                                          spike_margin=0.5)
    lut = orc.decode_fp8(np.arange(256, dtype=np.uint8)).astype(np.float64)
    D = q.shape[-1]
    for b in range(2):
        for h in range(8):
            kv = h // 4
            qs = q[b, h].astype(np.float32) * np.float32(1 / np.sqrt(np.float32(D)))
            fs = lut[c["far_k"][b, kv]] @ qs.astype(np.float64)
            ns = c["near_k"][b, kv, : nv[kv]].astype(np.float64) @ qs.astype(np.float64)
            ds = dk[b, kv].astype(np.float64) @ qs.astype(np.float64)
            assert tk[b, h] == int(np.argmax(fs))  # first index of the maximum
            mnear = min(ns.min(), ds.min())
            assert abs(mf[b, h] - fs.max()) < 1e-9 and abs(mn[b, h] - mnear) < 1e-9
            assert fl[b, h] == int(fs.max() > mnear + 0.5)


def test_formulation_oracle_brute_force(orc):
    rng = np.random.default_rng(2)
    c, q, nv, dk, dv = make_case(rng, orc=orc, B=1, Hq=8, Hkv=2, D=64, S=256, n_dec=3)
    out = orc.attend_formulation(q, c["near_k"], c["near_v"], nv, c["far_k"], c["far_v"],
                                 c["far_v_scale"], c["far_v_zero"], dk, dv)
    # the formulation orders near | decode | far; order does not change softmax
    bf = brute_force(q, c, nv, dk, dv, fp16_v=True)
    assert np.abs(out - bf).max() < 1e-9
    kern, *_ = orc.attend_kernel(q, c["near_k"], c["near_v"], nv, c["far_k"], c["far_v"],
                                 c["far_v_scale"], c["far_v_zero"], dk, dv)
    assert orc.cosine(out, kern) > 0.9999


def test_formulation_uses_max_near_valid(orc):
    """After uneven promotion the formulation slices near[:max(near_valid)]
    for every head (mlx_foveated.py:430-449); the kernel uses per-head counts."""
    rng = np.random.default_rng(4)
    c, q, nv, dk, dv = make_case(rng, orc=orc, B=1, Hq=4, Hkv=2, D=64, S=256, n_dec=0)
    nv2 = nv.copy()
    nv2[0] += 3  # head 0 has 3 promoted (zero) rows more than head 1
    f = orc.attend_formulation(q, c["near_k"], c["near_v"], nv2, c["far_k"], c["far_v"],
                               c["far_v_scale"], c["far_v_zero"])
    bf_max = brute_force(q, c, np.full_like(nv2, nv2.max()), None, None, fp16_v=True)
    assert np.abs(f - bf_max).max() < 1e-9


# ---------------------------------------------------------------------------
# importance partition (oracle.partition_importance)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("S", [0, 1, 3, 36, 37, 40, 100, 512, 1000, 4096])
def test_importance_equal_to_position_is_the_recency_partition(orc, S):
    n1, f1, _ = orc.tier_indices(S, 2, 3)
    n2, f2, _ = orc.partition_importance(np.arange(S, dtype=np.float32), S, 2, 3)
    assert np.array_equal(n1, n2) and np.array_equal(f1, f2)
    # a constant importance ties everywhere: ties go to the later token
    n3, f3, _ = orc.partition_importance(np.full(S, 0.5, np.float32), S, 2, 3)
    assert np.array_equal(n1, n3) and np.array_equal(f1, f3)


def test_importance_partition_brute_force_subsets(orc):
    """The chosen middle maximises (sum of importance, sum of positions)
    over every k-subset of the middle (exhaustive on small middles, integer
    importances with many ties)."""
    from itertools import combinations

    cfg = dict(near_pct=0.5, n_sinks=2, window_size=3)
    rng = np.random.default_rng(0)
    for S in (12, 17, 20):
        tb = orc.tier_boundaries(S, **cfg)
        mid = list(range(tb["mid_start"], tb["mid_end"]))
        k = tb["near_from_mid"]
        for trial in range(6):
            imp = rng.integers(0, 4, (1, 2, S)).astype(np.float32)
            near, far, _ = orc.partition_importance(imp, S, 1, 2, **cfg)
            for h in range(2):
                best = max(combinations(mid, k), key=lambda c: (sum(imp[0, h, list(c)]), sum(c)))
                got = near[0, h, tb["n_sinks"]:tb["n_sinks"] + k]
                assert list(got) == sorted(best), (S, trial, h)
                assert sorted(set(far[0, h]) | set(got)) == mid and len(far[0, h]) == len(mid) - k
                assert list(near[0, h, :tb["n_sinks"]]) == list(range(tb["n_sinks"]))
                assert list(near[0, h, tb["n_sinks"] + k:tb["R_actual"]]) == list(range(S - tb["window"], S))
                assert np.all(near[0, h, tb["R_actual"]:] == -1)


def test_importance_partition_special_values(orc):
    cfg = dict(near_pct=0.5, n_sinks=1, window_size=1)
    S = 12  # middle = positions 1..10, near_from_mid = 4
    imp = np.zeros(S, np.float32)
    imp[[2, 5]] = np.nan          # NaN ranks below everything, -inf included
    imp[3] = -np.inf
    imp[4] = np.inf
    imp[6] = -0.0                 # -0 == +0: ties with the zeros, later token wins
    imp[7] = 1.0
    near, far, tb = orc.partition_importance(imp, S, 1, 1, **cfg)
    assert tb["near_from_mid"] == 4
    assert list(near[0, 0, 1:5]) == [4, 7, 9, 10]
    assert list(far[0, 0]) == [1, 2, 3, 5, 6, 8]
    imp2 = np.full(S, np.nan, np.float32)
    imp2[1] = -np.inf
    near2, _, _ = orc.partition_importance(imp2, S, 1, 1, **cfg)
    assert list(near2[0, 0, 1:5]) == [1, 8, 9, 10]


def test_compress_with_position_importance_matches_recency(orc):
    rng = np.random.default_rng(3)
    k = rng.standard_normal((2, 2, 300, 64)).astype(np.float16)
    v = rng.standard_normal((2, 2, 300, 64)).astype(np.float16)
    a = orc.compress_layer(k, v)
    b = orc.compress_layer(k, v, importance=np.arange(300, dtype=np.float32))
    for n in ("near_k", "near_v", "far_k", "far_v", "far_v_scale", "far_v_zero", "archive_k", "archive_v",
              "near_idx", "far_idx"):
        assert np.array_equal(np.asarray(a[n]).view(np.uint8), np.asarray(b[n]).view(np.uint8)), n
