"""TurboQuant on the GPU through the C ABI, against the CPU restatement
(oracle/turbo.py, orc_attend_turbo): value codes bit-exact, key codes equal
wherever fp32 rounding cannot decide them, fused attention within max-abs
2e-3 and cosine 0.9999 of the kernel restatement, spikes equal."""

import numpy as np
import pytest
import torch

from _parity import record
from oracle import turbo as T

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _t(x, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(x)).to(DEV)
    return t if dtype is None else t.to(dtype)


def _stats(got, want):
    g = np.asarray(got, np.float64).ravel()
    w = np.asarray(want, np.float64).ravel()
    return float(np.max(np.abs(g - w))), float(g @ w / (np.linalg.norm(g) * np.linalg.norm(w) + 1e-30))


def _case(B, Hq, Hkv, D, F, Npad, nvalid, ndec, seed, spikes=0):
    rng = np.random.default_rng(seed)
    C = T.constants(D)
    kf = rng.standard_normal((B, Hkv, F, D)).astype(np.float16)
    vf = rng.standard_normal((B, Hkv, F, D)).astype(np.float16)
    q = rng.standard_normal((B, Hq, D)).astype(np.float16)
    g = Hq // Hkv
    for _ in range(spikes):  # far keys aligned with one query head: far scores well above the near minimum
        b, kv, t = rng.integers(B), rng.integers(Hkv), rng.integers(F)
        kf[b, kv, t] = (5 * q[b, kv * g].astype(np.float32)).astype(np.float16)
    idx, sg, nrm, gam = T.compress_keys(kf, C)
    vp, vs = T.compress_values(vf)
    L = dict(near_k=rng.standard_normal((B, Hkv, Npad, D)).astype(np.float16),
             near_v=rng.standard_normal((B, Hkv, Npad, D)).astype(np.float16),
             near_valid=np.asarray(nvalid, np.uint32), k_idx=idx, k_signs=sg, k_norm=nrm, k_gamma=gam,
             v_packed=vp, v_scale=vs,
             dec_k=rng.standard_normal((B, Hkv, ndec, D)).astype(np.float16) if ndec else None,
             dec_v=rng.standard_normal((B, Hkv, ndec, D)).astype(np.float16) if ndec else None)
    return C, q, L


def _handle(C, L, margin=10.0):
    from foveated_kv_amd.turbo import TurboFoveatedHandle

    return TurboFoveatedHandle(_t(L["near_k"]), _t(L["near_v"]), _t(L["k_idx"]), _t(L["k_signs"]),
                               _t(L["k_norm"]), _t(L["k_gamma"]), _t(L["v_packed"]), _t(L["v_scale"]),
                               _t(L["near_valid"].astype(np.int32)), torch.from_numpy(C["Pi"]),
                               torch.from_numpy(C["S"]), torch.from_numpy(C["centroids"]), spike_margin=margin)


def _run(h, q, L, q_dtype=torch.float16):
    qt = _t(q).to(q_dtype)[:, :, None, :]
    dk = _t(L["dec_k"]) if L["dec_k"] is not None else None
    dv = _t(L["dec_v"]) if L["dec_v"] is not None else None
    out, flags, toks = h(qt, dk, dv)
    torch.cuda.synchronize()
    return out[:, :, 0].float().cpu().numpy(), flags.cpu().numpy(), toks.cpu().numpy()


def _check_spikes(flags, toks, ref, q, L, C):
    """Equal except where the reference decision is within rounding: a far
    maximum tied (1e-3) with the score of the token the GPU chose, or
    max_far within 1e-3 of min_near + margin."""
    _, wf, wt, mf, mn = ref
    fs = T.far_scores(q, L["k_idx"], L["k_signs"], L["k_norm"], L["k_gamma"], C) if L["k_idx"].shape[2] else None
    for b, h in np.argwhere(toks != wt):
        assert fs is not None and 0 <= toks[b, h] < fs.shape[2], (b, h, toks[b, h])
        assert abs(fs[b, h, toks[b, h]] - fs[b, h, wt[b, h]]) < 1e-3, (b, h)
    for b, h in np.argwhere(flags != wf):
        assert abs(mf[b, h] - (mn[b, h] + 10.0)) < 1e-3, (b, h)


CASES = [
    # B, Hq, Hkv, D, F, Npad, nvalid, ndec
    (1, 8, 2, 128, 300, 70, (64, 50), 5),
    (2, 32, 8, 128, 1900, 210, tuple(range(150, 206, 7)), 17),
    (1, 14, 2, 64, 461, 76, (51, 51), 16),
    (1, 16, 1, 128, 1000, 128, (100,), 0),
    (2, 4, 4, 64, 129, 64, (64, 10, 0, 33), 3),
    (1, 8, 2, 128, 0, 64, (40, 64), 2),
    (2, 24, 2, 128, 8000, 896, (800, 750), 4),  # G = 12: rows of three head quads
    (1, 28, 4, 128, 9000, 1000, (900, 850, 1000, 700), 3),  # G = 7: 16-head rows, second quad partial
]


@pytest.mark.parametrize("cfg", CASES, ids=[f"B{c[0]}_Hq{c[1]}_Hkv{c[2]}_D{c[3]}_F{c[4]}" for c in CASES])
def test_turbo_attention_matches_kernel_restatement(cfg):
    B, Hq, Hkv, D, F, Npad, nv, nd = cfg
    print("case:", cfg, flush=True)
    C, q, L = _case(B, Hq, Hkv, D, F, Npad, nv, nd, seed=sum(cfg[:5]), spikes=3 if F else 0)
    ref = T.attend_kernel(q, **L, C=C)
    h = _handle(C, L)
    out, flags, toks = _run(h, q, L)
    mx, cs = _stats(out, ref[0])
    assert mx <= 2e-3 and cs >= 0.9999, (mx, cs)
    _check_spikes(flags, toks, ref, q, L, C)


def test_turbo_query_dtypes_and_back_to_back_calls():
    C, q, L = _case(2, 16, 4, 128, 700, 96, (80, 60, 96, 10), 9, seed=21, spikes=2)
    ref = T.attend_kernel(q, **L, C=C)
    h = _handle(C, L)
    first = _run(h, q, L)
    for dt in (torch.bfloat16, torch.float32):
        qd = _t(q).to(dt).float().cpu().numpy().astype(np.float16)  # the kernel casts the query to fp16
        r = T.attend_kernel(qd, **L, C=C) if dt == torch.bfloat16 else ref
        out, flags, toks = _run(h, q if dt == torch.float32 else qd, L, q_dtype=dt)
        mx, cs = _stats(out, r[0])
        assert mx <= 2e-3 and cs >= 0.9999, (dt, mx, cs)
    for _ in range(20):
        again = _run(h, q, L)
        assert np.array_equal(again[0], first[0]) and np.array_equal(again[1], first[1])


def test_turbo_general_centroids():
    """Asymmetric centroids exercise the constant and cross terms of the
    centroid decomposition (alpha, delta != 0)."""
    C, q, L = _case(1, 8, 2, 128, 500, 64, (64, 30), 4, seed=5)
    C2 = dict(C)
    C2["centroids"] = np.array([-0.11, -0.05, 0.02, 0.16], np.float32)
    ref = T.attend_kernel(q, **L, C=C2)
    out, _, _ = _run(_handle(C2, L), q, L)
    mx, cs = _stats(out, ref[0])
    assert mx <= 2e-3 and cs >= 0.9999, (mx, cs)


def test_turbo_compress_values_bit_exact():
    rng = np.random.default_rng(1)
    from foveated_kv_amd.turbo import turbo_compress_values

    for D in (64, 128):
        v = rng.standard_normal((2, 3, 77, D)).astype(np.float16)
        v[0, 0, 0, :32] = 0.0  # all-zero group: scale half(1e-8) = 0, codes 2
        v[0, 0, 1, :8] = [3, -3, 1, -1, 0, 0.5, 2, -2]  # (2/3 + 1) * 1.5 == 2.5 in fp32: half to even
        v[0, 0, 1, 8:32] = 0.25
        want_p, want_s = T.compress_values(v)
        for dt in (torch.float16, torch.float32):
            p, s = turbo_compress_values(_t(v).to(dt))
            assert np.array_equal(p.cpu().numpy(), want_p), (D, dt)
            assert np.array_equal(s.cpu().numpy().view(np.uint16), want_s.view(np.uint16)), (D, dt)


def test_turbo_compress_keys_matches_restatement():
    from foveated_kv_amd.turbo import get_turbo_constants, turbo_compress_keys

    rng = np.random.default_rng(2)
    for D in (64, 128):
        C = T.constants(D)
        k = rng.standard_normal((2, 3, 150, D)).astype(np.float16)
        k[0, 0, 0] = 0  # zero key: norm 0, every rotated coordinate 0
        idx, sg, nrm, gam, ymarg, pmarg, codes, bits = T.compress_keys(k, C, margins=True)
        gi, gs, gn, gg = turbo_compress_keys(_t(k), get_turbo_constants(D))
        gcodes = T.unpack_2bit(gi.cpu().numpy())
        gbits = (T.unpack_1bit(gs.cpu().numpy()) > 0).astype(np.uint8)
        # a code may differ only where the fp64 rotated coordinate lies within
        # 1e-6 of a boundary: the fp32 rotation of a unit vector (|y| <= 1,
        # sum_j |k_j Pi_ij| / |k| <= 1) is off by ~sqrt(D) * 2^-24 << 1e-6
        loose_c = ymarg < 1e-6
        loose_s = pmarg < 1e-4
        assert np.array_equal(gcodes[~loose_c], codes[~loose_c]), D
        assert np.array_equal(gbits[~loose_s], bits[~loose_s]), D
        assert loose_c.mean() < 5e-3 and loose_s.mean() < 5e-3  # the zero key alone is 1/900 of the codes
        record(f"TurboQuant key compression D={D} (2x3x150 keys)", codes=int(loose_c.size),
               loose_codes=int(loose_c.sum()), differing_codes=int((gcodes != codes).sum()),
               loose_signs=int(loose_s.sum()), differing_signs=int((gbits != bits).sum()))
        n32, g32 = gn.float().cpu().numpy(), gg.float().cpu().numpy()
        assert np.allclose(n32, nrm.astype(np.float32), rtol=1e-3, atol=0)
        assert np.allclose(g32, gam.astype(np.float32), rtol=2e-3, atol=1e-3)


def test_turbo_cache_layer_fused_against_formulation_and_restatement():
    from foveated_kv_amd import MLXFoveatedKVCache, MLXTierConfig

    rng = np.random.default_rng(4)
    B, H, S, D, Hq = 1, 2, 1024, 128, 8
    keys = _t(rng.standard_normal((B, H, S, D)).astype(np.float16))
    vals = _t(rng.standard_normal((B, H, S, D)).astype(np.float16))
    cache = MLXFoveatedKVCache(MLXTierConfig(compress_method="turbo"))
    cache.update(keys, vals, 0)
    cache.compress()
    lay = cache.layers[0]
    assert lay.compress_method == "turbo" and lay.far_k.shape[2] == 0
    assert lay.turbo_far_k_indices.shape == (B, H, lay.far_idx.shape[2], D // 4)
    lay.add_token(_t(rng.standard_normal((B, H, 1, D)).astype(np.float16)),
                  _t(rng.standard_normal((B, H, 1, D)).astype(np.float16)))
    q = _t(rng.standard_normal((B, Hq, 1, D)).astype(np.float16))
    fused = lay.attend_fused(q).float()
    form = lay.attend(q).float()
    a, b = fused.cpu().numpy().ravel(), form.cpu().numpy().ravel()
    assert a @ b / (np.linalg.norm(a) * np.linalg.norm(b)) > 0.97  # the reference's two turbo paths differ
    n = lambda t: t.cpu().numpy()
    C = T.constants(D)
    ref = T.attend_kernel(n(q[:, :, 0]), n(lay.near_k), n(lay.near_v), n(lay.near_valid).astype(np.uint32),
                          n(lay.turbo_far_k_indices), n(lay.turbo_far_k_signs), n(lay.turbo_far_k_norm),
                          n(lay.turbo_far_k_gamma), n(lay.turbo_far_v_packed), n(lay.turbo_far_v_scale), C,
                          dec_k=n(lay.decode_k), dec_v=n(lay.decode_v))
    mx, cs = _stats(fused[:, :, 0].cpu().numpy(), ref[0])
    assert mx <= 2e-3 and cs >= 0.9999, (mx, cs)
