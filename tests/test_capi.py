"""C-ABI checks that need no GPU: the library loads, exports exactly what
include/fkv.h declares, and its host-only entry points behave."""

import ctypes
import os
import re

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared_functions():
    names = set()
    for fn in os.listdir(os.path.join(ROOT, "include")):
        if fn.endswith(".h"):
            text = open(os.path.join(ROOT, "include", fn)).read()
            text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
            names |= set(re.findall(r"\b(fkv_[a-z0-9_]+)\s*\(", text))
    return names


def test_library_exports_every_declared_symbol():
    from foveated_kv_amd import _lib

    lib = _lib.load()
    declared = _declared_functions()
    assert declared, "no declarations parsed"
    for name in declared:
        assert hasattr(lib, name), f"{name} declared in include/ but not exported"
    # the Python binding covers every declared symbol
    assert declared == set(_lib.SIGNATURES), declared ^ set(_lib.SIGNATURES)
    out = os.popen(f"nm -D --defined-only {_lib.LIB_PATH}").read()
    exported = set(re.findall(r"\bT (fkv_[a-z0-9_]+)\b", out))
    assert declared <= exported


def test_version_and_error_channel():
    from foveated_kv_amd import _lib

    lib = _lib.load()
    assert lib.fkv_version() >= 100
    # NULL config -> error code + message, no crash
    rc = lib.fkv_tier_boundaries(None, 10, None)
    assert rc == _lib.FKV_EINVAL
    assert b"fkv_tier_boundaries" in lib.fkv_last_error()
    # bad shapes rejected before any device work
    h = ctypes.c_void_p()
    rc = lib.fkv_attn_create(ctypes.byref(h), 1, 1, 96, 8, 8, None, None, 0, None, None, None, None, 0,
                             None, 0.5, None)
    assert rc == _lib.FKV_EINVAL and b"64 or 128" in lib.fkv_last_error()
    rc = lib.fkv_attn_call(None, None, 0, 1, None, None, 0, None, None, None, None)
    assert rc == _lib.FKV_EINVAL


@pytest.mark.parametrize("S", [0, 1, 4, 36, 37, 100, 512, 1000, 4096, 16384, 32768, 65536, 100003])
@pytest.mark.parametrize("pct,hmin", [(0.10, 8), (0.25, 4), (0.05, 0), (0.5, 8)])
def test_tier_boundaries_c_matches_oracle_and_python(orc, S, pct, hmin):
    from foveated_kv_amd import TierConfig, ext

    c = ext.TierConfig()
    c.near_pct = pct
    c.promo_headroom_min = hmin
    got = ext.tier_boundaries_c(c, S)
    ref = orc.tier_boundaries(S, near_pct=pct, promo_headroom_min=hmin)
    py = TierConfig(near_pct=pct, promo_headroom_min=hmin).tier_boundaries(S)
    for key in ref:
        assert got[key] == ref[key], key
    for key in py:
        assert py[key] == ref[key], key


def test_tier_config_validation():
    from foveated_kv_amd import MLXTierConfig, TierConfig

    assert MLXTierConfig is TierConfig
    with pytest.raises(ValueError, match="compress_method"):
        TierConfig(compress_method="invalid")
    assert TierConfig().compress_method == "fp8"
    from foveated_kv_amd import ext

    assert ext.TierConfig().promo_headroom_min == 4  # C++ default, foveated_compress.h:97


def test_cpu_tensors_are_rejected():
    import torch

    from foveated_kv_amd import ext

    x = torch.zeros((1, 1, 8, 64), dtype=torch.float16)
    with pytest.raises(TypeError, match="ROCm device"):
        ext.CompressHandle().compress_layer(x, x)


def test_missing_library_fails_loudly(tmp_path, monkeypatch):
    from foveated_kv_amd import _lib

    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(_lib, "_load_error", None)
    monkeypatch.setattr(_lib, "LIB_PATH", str(tmp_path / "libfkv.so"))
    with pytest.raises(_lib.FkvLibraryError, match="not built"):
        _lib.load()
    from foveated_kv_amd import ext

    assert ext.is_available() is False


def _far_plan(lib, N, NT, FT, NB, FB, turbo):
    f0 = (ctypes.c_int32 * N)()
    fs = (ctypes.c_int32 * N)()
    nf = (ctypes.c_int32 * N)()
    assert lib.fkv_far_plan(N, NT, FT, NB, FB, turbo, f0, fs, nf) == 0
    return list(f0), list(fs), list(nf)


def test_far_plan_covers_every_far_tile_once():
    """The attention kernel's per-wave far-tile plan (the same function the
    kernel runs): over random row shapes every far tile is streamed by
    exactly one wave; outside TurboQuant's round-robin regime the waves take
    contiguous, ordered ranges."""
    import random

    from foveated_kv_amd import _lib

    lib = _lib.load()
    rng = random.Random(11)
    shapes = [(16, 26, 231), (16, 13, 116), (16, 52, 461), (128, 103, 922), (32, 10, 58), (4, 2, 8), (8, 0, 5),
              (64, 300, 3), (256, 0, 0)]
    shapes += [(rng.choice([4, 8, 12, 16, 32, 64, 128, 256]), rng.randint(0, 400), rng.randint(0, 4000))
               for _ in range(1500)]
    for N, NT, FT in shapes:
        for NB, FB, turbo in ((256 * 128, 12544, 0), (128 * 128, 12544, 0), (256 * 64, 6272, 0),
                              (256 * 128, 13312, 0), (256 * 128, 5888, 1), (256 * 64, 2944 + 256, 1)):
            f0, fs, nf = _far_plan(lib, N, NT, FT, NB, FB, turbo)
            tiles = [f0[w] + u * fs[w] for w in range(N) for u in range(nf[w])]
            assert sorted(tiles) == list(range(FT)), (N, NT, FT, NB, FB, turbo)
            if all(s == 1 for s in fs):
                assert all(f0[w] + nf[w] == f0[w + 1] for w in range(N - 1)), (N, NT, FT, NB, FB, turbo)
            elif not turbo:
                pytest.fail(f"round-robin far plan outside TurboQuant: {(N, NT, FT, NB, FB)}")


def test_far_plan_balances_c3_16k():
    """C3-16K (16 waves per row, 26 near and 231 far tiles of 12,544 bytes,
    near tiles round-robin): every wave's bytes within one far tile of the
    mean, the worst within 0.6 of one."""
    from foveated_kv_amd import _lib

    lib = _lib.load()
    N, NT, FT, NB, FB = 16, 26, 231, 256 * 128, 12544
    f0, fs, nf = _far_plan(lib, N, NT, FT, NB, FB, 0)
    cost = [(NT // N + (1 if w < NT % N else 0)) * NB + nf[w] * FB for w in range(N)]
    mean = sum(cost) / N
    assert max(abs(c - mean) for c in cost) <= FB
    assert max(cost) - mean <= 0.6 * FB
    with pytest.raises(Exception):
        _lib.check(lib.fkv_far_plan(0, 1, 1, NB, FB, 0, None, None, None), "fkv_far_plan")


@pytest.mark.parametrize("fmt", [0, 1, 2])
@pytest.mark.parametrize("B,Hkv,D,S,Hq", [
    (8, 8, 128, 16384, 32), (8, 8, 128, 32768, 32), (1, 8, 128, 65536, 64), (1, 2, 64, 512, 14),
    (1, 8, 128, 4096, 32), (1, 2, 64, 600, 12), (4, 2, 128, 4096, 40), (1, 4, 128, 40, 24), (3, 4, 64, 333, 12),
    (1, 1, 64, 100, 1), (2, 2, 128, 9000, 96), (4, 8, 128, 8192, 32),
])
def test_launch_plan_never_outgrows_the_first_call_workspace(orc, B, Hkv, D, S, Hq, fmt):
    """A handle's workspace is allocated once, by its first call, and never
    re-allocated (a captured HIP graph keeps its pointers): every decode
    length and split target must plan within it, for every far format
    (TurboQuant rows of one head quad at D = 128 run 8 waves, so up to 32
    wave records per row)."""
    from foveated_kv_amd import _lib

    lib = _lib.load()
    tb = orc.tier_boundaries(S)
    Na, F = tb["N_near_padded"], tb["far_count"]
    out = (ctypes.c_int64 * 8)()
    worst, eight = 0, False
    for n_dec in list(range(0, 130)) + [255, 256, 257, 1000, 4096, 70000]:
        for target in (1, 64, 256, 1024, 4096):
            assert lib.fkv_attn_plan(B, Hkv, D, Na, F, Hq, n_dec, target, fmt, out) == _lib.FKV_OK
            hpg, rows, splits, need, have, rows_have, waves, recs = list(out)
            assert hpg in (4, 16) and 1 <= splits <= 64
            assert waves == (8 if fmt == 1 and D == 128 and min(hpg, Hq // Hkv) <= 4 else 4)
            assert recs in (1, waves) and splits * recs <= 64  # the merge reads at most kMaxSplits records
            assert rows <= rows_have, (n_dec, target, rows, rows_have)
            assert need <= have, (n_dec, target, need, have)
            worst = max(worst, need)
            eight |= waves == 8 and recs == 8
    assert worst > 0 or Na + F < 2 * 64 * 4
    if fmt == 1 and D == 128 and Hq // Hkv <= 4 and Na + F > 8 * 64 * 16:
        assert eight  # some plan keeps 8 wave records per split (32 per row)
    assert lib.fkv_attn_plan(B, Hkv, D, Na, F, Hq + 1 if Hkv > 1 else 0, 0, 256, fmt, out) == _lib.FKV_EINVAL
    assert lib.fkv_attn_plan(B, Hkv, D, Na, F, Hq, 0, 256, 3, out) == _lib.FKV_EINVAL


def test_xcd_rule_fit_and_watch_words():
    """The host logic of the XCD-local merge's two checks: the dispatch rule
    fitted to a probe's XCD ids (workgroup i on lo + (c + i) mod X), and the
    violations a watch-word array holds."""
    from foveated_kv_amd import _lib

    lib = _lib.load()

    def fit(ids):
        a = np.ascontiguousarray(ids, np.uint32)
        X, c = _lib.I32(-1), _lib.I32(-1)
        assert lib.fkv_xcd_rule_fit(a.ctypes.data_as(ctypes.c_void_p), a.size, ctypes.byref(X), ctypes.byref(c)) == 0
        return X.value, c.value

    n = 4096
    assert fit([(7 + i) % 8 for i in range(n)]) == (8, 7)
    assert fit([(i % 8) for i in range(n)]) == (8, 0)
    assert fit([2 + (3 + i) % 4 for i in range(n)]) == (4, 3)   # ids 2..5
    assert fit([5] * n) == (1, 0)
    broken = [(7 + i) % 8 for i in range(n)]
    broken[1000], broken[1001] = broken[1001], broken[1000]
    assert fit(broken) == (0, 0)
    assert fit([(i // 2) % 8 for i in range(n)]) == (0, 0)      # pairs per XCD: not round-robin

    def viol(words):
        a = np.ascontiguousarray(words, np.uint32)
        return lib.fkv_xcd_watch_violations(a.ctypes.data_as(ctypes.c_void_p), a.size - 1)

    assert viol([0] * 65) == 0
    assert viol([1] + [0] * 64) == 1                 # a merge saw another XCD's record
    assert viol([0, 0, 3, 0, 1]) == 2                # counters no merge re-armed
    assert viol([1, 2]) == 2
