"""fkv_attn_call_noalloc: the attention call that allocates nothing (its
workspace is a fixed device array per GPU), through the C ABI, against
fkv_attn_call on the same handles -- same kernels, same launch plan, so the
outputs must be the same bits -- and against the CPU oracle within the
parity tolerance.  Two calls in a row, the second with a smaller input
(another shape, a bf16 query), then the first again; the first call on a
fresh handle leaves the device's free memory unchanged; a call whose plan
does not fit the array (too many rows, or rows whose split records exceed
it) is refused before any GPU work."""

import ctypes

import numpy as np
import pytest
import torch

from _parity import ATOL, COS, flush, np_, tier_config

pytestmark = pytest.mark.gpu


def _case(B, Hq, Hkv, D, S, n_dec, seed, spikes=0.0):
    from foveated_kv_amd import ext, synthetic

    k, v = synthetic.make_kv(B, Hkv, S, D, seed)
    q = synthetic.make_query(B, Hq, D, seed)
    tb = ext.tier_boundaries_c(tier_config(), S)
    synthetic.inject_spikes(k, q, tb["mid_start"], tb["far_count"], spikes, seed)
    dk, dv = synthetic.make_decode(B, Hkv, n_dec, D, seed)
    cl = ext.CompressHandle(tier_config()).compress_layer(torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda(),
                                                         with_archive=False)
    h = ext.FoveatedHandle(cl.near_k, cl.near_v, cl.far_k, cl.far_v, cl.far_v_scale, cl.far_v_zero,
                           cl.near_valid, spike_margin=10.0)
    c = {n: np_(getattr(cl, n)) for n in ("near_k", "near_v", "far_k", "far_v", "far_v_scale", "far_v_zero",
                                          "near_valid")}
    return h, q, dk, dv, c


def _call(entry, h, q, dk, dv):
    """One call through the C ABI into preallocated outputs."""
    from foveated_kv_amd import _lib

    B, Hq, D = q.shape
    out = torch.empty((B, Hq, D), dtype=torch.float16, device="cuda")
    flags = torch.empty((B, Hq), dtype=torch.int32, device="cuda")
    toks = torch.empty((B, Hq), dtype=torch.int32, device="cuda")
    n_dec = dk.shape[2] if dk is not None else 0
    rc = getattr(_lib.load(), entry)(h._h, _lib.ptr(q), _lib.dtype_code(q.dtype), Hq, _lib.ptr(dk), _lib.ptr(dv),
                                     n_dec, _lib.ptr(out), _lib.ptr(flags), _lib.ptr(toks), _lib.stream_ptr())
    _lib.check(rc, entry)
    return out, flags, toks


def _check(orc, h, q, dk, dv, c, q_dtype, what):
    qt = torch.from_numpy(q).cuda().to(q_dtype)
    dkt = torch.from_numpy(dk).cuda() if dk is not None else None
    dvt = torch.from_numpy(dv).cuda() if dv is not None else None
    got = _call("fkv_attn_call_noalloc", h, qt, dkt, dvt)
    want = _call("fkv_attn_call", h, qt, dkt, dvt)
    torch.cuda.synchronize()
    for x, y, n in zip(got, want, ("out", "flags", "tokens")):
        assert torch.equal(x, y), f"{what}: {n} differs from fkv_attn_call"
    ko = orc.attend_kernel(np_(qt.to(torch.float16)), c["near_k"], c["near_v"], c["near_valid"], c["far_k"],
                           c["far_v"], c["far_v_scale"], c["far_v_zero"], dk, dv, spike_margin=10.0)[0]
    out = np_(got[0]).astype(np.float64)
    err, cos = float(np.abs(out - ko).max()), orc.cosine(out, ko)
    flush(f"  {what}: max-abs {err:.3e} cos {cos:.8f} vs the oracle")
    assert err <= ATOL and cos >= COS
    return [t.clone() for t in got]


def test_noalloc_matches_allocating_call(orc):
    flush("no-alloc call 1: B=4 Hq=32 Hkv=8 D=128 S=8192 n_dec=64, 2 % spikes")
    big = _case(4, 32, 8, 128, 8192, 64, seed=501, spikes=0.02)
    first = _check(orc, *big, torch.float16, "call 1 (larger)")
    flush("no-alloc call 2 (smaller): B=1 Hq=14 Hkv=2 D=64 S=512 n_dec=16, bf16 query")
    small = _case(1, 14, 2, 64, 512, 16, seed=502)
    _check(orc, *small, torch.bfloat16, "call 2 (smaller, bf16 query)")
    flush("no-alloc call 3: call 1 again on the shared scratch")
    again = _check(orc, *big, torch.float16, "call 3 (call 1 again)")
    for x, y in zip(first, again):
        assert torch.equal(x, y)


def test_noalloc_first_call_on_a_fresh_handle_allocates_nothing(orc):
    """fkv_attn_call would size a ~35 MB split workspace on this handle's
    first call; the no-alloc entry point must leave the device's free memory
    as it was (the kernels and the scratch array are loaded by a call on
    another handle first)."""
    flush("no-alloc fresh handle: B=4 Hq=32 Hkv=8 D=128 S=8192")
    warm = _case(1, 14, 2, 64, 512, 16, seed=503)
    _check(orc, *warm, torch.float16, "warm-up call (another handle)")
    h, q, dk, dv, c = _case(4, 32, 8, 128, 8192, 0, seed=504)
    qt = torch.from_numpy(q).cuda()
    torch.cuda.synchronize()
    free0 = torch.cuda.mem_get_info()[0]
    got = _call("fkv_attn_call_noalloc", h, qt, None, None)
    torch.cuda.synchronize()
    free1 = torch.cuda.mem_get_info()[0]
    assert free1 == free0, f"free device memory changed by {free0 - free1} bytes"
    ko = orc.attend_kernel(q, c["near_k"], c["near_v"], c["near_valid"], c["far_k"], c["far_v"],
                           c["far_v_scale"], c["far_v_zero"], spike_margin=10.0)[0]
    out = np_(got[0]).astype(np.float64)
    assert float(np.abs(out - ko).max()) <= ATOL and orc.cosine(out, ko) >= COS


def test_noalloc_refuses_records_beyond_its_scratch():
    """Rows that fit the counter region (128) but whose split records do
    not fit the array: B=64 x 2 KV heads of 16-head rows, 2 splits x 4 wave
    records x 16 heads x 136 floats = 8.5 MiB of records (9.06 MiB with the
    counters and the query copy, fkv_attn_plan): refused before any GPU
    work."""
    from foveated_kv_amd import _lib, ext

    B, Hkv, Hq, D, S = 64, 2, 32, 128, 1024
    cfg = tier_config()
    tb = ext.tier_boundaries_c(cfg, S)
    lib = _lib.load()
    plan = (ctypes.c_int64 * 8)()
    assert lib.fkv_attn_plan(B, Hkv, D, tb["N_near_padded"], tb["far_count"], Hq, 0, 256, 0, plan) == 0
    assert plan[0] == 16 and plan[1] == 128 and plan[2] == 2
    qbytes = (B * Hq * D * 2 + 255) // 256 * 256
    assert 65536 + qbytes + plan[3] * 4 > 8 << 20 and plan[1] * 4 <= 65536
    nk = torch.zeros((B, Hkv, tb["N_near_padded"], D), dtype=torch.float16, device="cuda")
    F = tb["far_count"]
    fk = torch.zeros((B, Hkv, F, D), dtype=torch.uint8, device="cuda")
    fv = torch.zeros((B, Hkv, F, D // 2), dtype=torch.uint8, device="cuda")
    sc = torch.ones((B, Hkv, F), dtype=torch.float16, device="cuda")
    h = ext.FoveatedHandle(nk, nk, fk, fv, sc, sc, torch.full((Hkv,), tb["R_actual"], dtype=torch.int32,
                                                              device="cuda"))
    q = torch.zeros((B, Hq, D), dtype=torch.float16, device="cuda")
    out = torch.empty((B, Hq, D), dtype=torch.float16, device="cuda")
    fl = torch.empty((B, Hq), dtype=torch.int32, device="cuda")
    rc = lib.fkv_attn_call_noalloc(h._h, _lib.ptr(q), _lib.FKV_F16, Hq, None, None, 0, _lib.ptr(out), _lib.ptr(fl),
                                   _lib.ptr(fl), _lib.stream_ptr())
    assert rc == _lib.FKV_EINVAL
    assert b"no-alloc entry point holds" in lib.fkv_last_error()


def test_noalloc_refuses_a_plan_beyond_its_scratch():
    """16,800 rows of arrival counters exceed the array's 16,384: refused
    with a clear message before any GPU work (no far tier, tiny near tier)."""
    from foveated_kv_amd import _lib, ext

    B, Hkv, Hq, D, Na = 4200, 4, 4, 64, 8
    nk = torch.zeros((B, Hkv, Na, D), dtype=torch.float16, device="cuda")
    fk = torch.zeros((B, Hkv, 0, D), dtype=torch.uint8, device="cuda")
    fv = torch.zeros((B, Hkv, 0, D // 2), dtype=torch.uint8, device="cuda")
    sc = torch.zeros((B, Hkv, 0), dtype=torch.float16, device="cuda")
    h = ext.FoveatedHandle(nk, nk, fk, fv, sc, sc, torch.full((Hkv,), Na, dtype=torch.int32, device="cuda"))
    q = torch.zeros((B, Hq, D), dtype=torch.float16, device="cuda")
    lib = _lib.load()
    out = torch.empty((B, Hq, D), dtype=torch.float16, device="cuda")
    fl = torch.empty((B, Hq), dtype=torch.int32, device="cuda")
    rc = lib.fkv_attn_call_noalloc(h._h, _lib.ptr(q), _lib.FKV_F16, Hq, None, None, 0, _lib.ptr(out), _lib.ptr(fl),
                                   _lib.ptr(fl), _lib.stream_ptr())
    assert rc == _lib.FKV_EINVAL
    assert b"no-alloc entry point holds" in lib.fkv_last_error()
