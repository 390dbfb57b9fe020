"""Importance partition and indexed compression on the GPU (through the C
ABI) against the oracle: index sets and every compressed byte bit-exact;
importance = position reproduces the recency partition byte for byte."""

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _np(t):
    return t.detach().cpu().numpy()


def _cfg(v_group=0, **kw):
    from foveated_kv_amd import ext

    c = ext.TierConfig()
    c.promo_headroom_min = 8
    c.v_group = v_group
    for k, v in kw.items():
        setattr(c, k, v)
    return c


def _importance(rng, B, H, S, kind):
    if kind == "ties":  # few distinct values: most of the decision is the tie rule
        return rng.integers(0, 5, (B, H, S)).astype(np.float32)
    imp = rng.standard_normal((B, H, S)).astype(np.float32)
    if kind == "special":
        n = imp.size
        flat = imp.reshape(-1)
        flat[rng.integers(0, n, n // 20)] = np.nan
        flat[rng.integers(0, n, n // 50)] = np.inf
        flat[rng.integers(0, n, n // 50)] = -np.inf
        flat[rng.integers(0, n, n // 20)] = -0.0
        flat[rng.integers(0, n, n // 20)] = 0.0
    return imp


@pytest.mark.parametrize("B,H,S,kind", [
    (1, 2, 512, "normal"), (2, 3, 1000, "ties"), (1, 8, 65536, "normal"), (2, 2, 4096, "special"),
    (1, 1, 37, "normal"), (1, 2, 40, "ties"), (1, 1, 3, "normal"), (3, 2, 2049, "ties"),
])
def test_partition_bit_exact(orc, B, H, S, kind):
    from foveated_kv_amd import ext

    print(f"partition B={B} H={H} S={S} {kind}", flush=True)
    imp = _importance(np.random.default_rng(S + B), B, H, S, kind)
    near, far = ext.partition_importance(_cfg(), torch.from_numpy(imp).cuda(), B, H, S)
    torch.cuda.synchronize()
    wn, wf, _ = orc.partition_importance(imp, S, B, H)
    assert np.array_equal(_np(near), wn)
    assert np.array_equal(_np(far), wf)


def test_partition_other_tier_configs(orc):
    from foveated_kv_amd import ext

    rng = np.random.default_rng(9)
    for kw in (dict(n_sinks=0, window_size=0), dict(near_pct=0.5), dict(near_pct=0.0), dict(near_pct=1.0)):
        imp = rng.standard_normal((1, 2, 777)).astype(np.float32)
        near, far = ext.partition_importance(_cfg(**kw), torch.from_numpy(imp).cuda(), 1, 2, 777)
        torch.cuda.synchronize()
        wn, wf, _ = orc.partition_importance(imp, 777, 1, 2, promo_headroom_min=8, **kw)
        assert np.array_equal(_np(near), wn), kw
        assert np.array_equal(_np(far), wf), kw


@pytest.mark.parametrize("B,H,S,D,vg", [(1, 2, 512, 64, 0), (2, 3, 1000, 128, 0), (1, 2, 700, 128, 32),
                                        (1, 1, 37, 64, 32)])
def test_indexed_compress_bit_exact(orc, B, H, S, D, vg):
    from foveated_kv_amd import ext, synthetic

    print(f"indexed compress B={B} H={H} S={S} D={D} v_group={vg}", flush=True)
    k, v = synthetic.make_kv(B, H, S, D, seed=S)
    imp = _importance(np.random.default_rng(S), B, H, S, "normal")
    cl = ext.CompressHandle(_cfg(vg)).compress_layer(torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda(),
                                                     importance=torch.from_numpy(imp).cuda())
    torch.cuda.synchronize()
    ref = orc.compress_layer(k, v, v_group=vg, importance=imp)
    for n in ("near_k", "near_v", "far_k", "far_v", "far_v_scale", "far_v_zero", "archive_k", "archive_v",
              "near_idx", "far_idx", "near_valid"):
        got, want = _np(getattr(cl, n)), np.asarray(ref[n])
        assert got.shape == want.shape, n
        assert np.array_equal(got.view(np.uint8), want.astype(got.dtype).view(np.uint8)), n


def test_position_importance_equals_recency_compress():
    from foveated_kv_amd import ext, synthetic

    k, v = synthetic.make_kv(2, 2, 1500, 128, seed=4)
    kt, vt = torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda()
    h = ext.CompressHandle(_cfg())
    a = h.compress_layer(kt, vt)
    b = h.compress_layer(kt, vt, importance=torch.arange(1500, dtype=torch.float32, device="cuda"))
    for n in ("near_k", "near_v", "far_k", "far_v", "far_v_scale", "far_v_zero", "archive_k", "archive_v"):
        assert torch.equal(getattr(a, n), getattr(b, n)), n


def test_cache_with_importance_fused_matches_formulation(orc):
    from foveated_kv_amd import MLXFoveatedKVCache, MLXTierConfig

    rng = np.random.default_rng(5)
    B, H, S, D, Hq = 1, 2, 2048, 128, 8
    keys = torch.from_numpy(rng.standard_normal((B, H, S, D)).astype(np.float16)).cuda()
    vals = torch.from_numpy(rng.standard_normal((B, H, S, D)).astype(np.float16)).cuda()
    imp = torch.from_numpy(rng.standard_normal((B, H, S)).astype(np.float32)).cuda()
    cache = MLXFoveatedKVCache(MLXTierConfig())
    cache.update(keys, vals, 0)
    cache.compress(importance=imp)
    lay = cache.layers[0]
    assert not torch.equal(lay.far_idx[0, 0], lay.far_idx[0, 1])  # per-head partitions
    q = torch.from_numpy(rng.standard_normal((B, Hq, 1, D)).astype(np.float16)).cuda()
    fused = lay.attend_fused(q).float().cpu().numpy()
    form = lay.attend(q).float().cpu().numpy()
    assert np.abs(fused - form).max() <= 2e-3 and orc.cosine(fused, form) >= 0.9999
    # exact attention over the original rows: the near tier holds the chosen tokens
    ni = _np(lay.near_idx[0, 0])
    assert np.array_equal(_np(lay.near_k[0, 0, :int(lay.near_valid[0])]),
                          _np(keys[0, 0, ni[ni >= 0].astype(np.int64)]))
