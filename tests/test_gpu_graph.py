"""Decode-buffer length kept on the device (fkv_attn_call_dev) and a decode
step captured in a HIP graph: the same bits as the host-count call.

The device-count entry point reads the number of valid rows of a
fixed-capacity decode buffer inside the kernel, so one captured launch
serves every step while the buffer fills.  With the same split plan the
work partition is identical, so outputs, spike flags and spike tokens must
equal the host-count call's exactly; the host-count call itself is held to
the oracle by the parity tests.
"""

import pytest
import torch

pytestmark = pytest.mark.gpu


def _flush(msg):
    print(msg, flush=True)


@pytest.fixture(scope="module")
def fkv():
    import foveated_kv_amd
    from foveated_kv_amd import _lib

    _lib.load()
    assert torch.cuda.is_available(), "GPU tests need a ROCm device"
    assert foveated_kv_amd.is_available(), "libfkv.so loaded but no gfx950 device"
    return foveated_kv_amd


def _layer(B, Hq, Hkv, D, S, seed, v_group=0):
    """A compressed layer (S = 8192 keeps the split plan independent of the
    decode rows: the per-row tile cap stays above the occupancy target)."""
    from foveated_kv_amd import ext, synthetic

    k, v = synthetic.make_kv(B, Hkv, S, D, seed)
    cfg = ext.TierConfig()
    cfg.promo_headroom_min = 8
    cfg.v_group = v_group
    cl = ext.CompressHandle(cfg).compress_layer(torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda(),
                                               with_archive=False)
    h = ext.FoveatedHandle(cl.near_k, cl.near_v, cl.far_k, cl.far_v, cl.far_v_scale, cl.far_v_zero,
                           cl.near_valid, spike_margin=10.0)
    q = torch.from_numpy(synthetic.make_query(B, Hq, D, seed)).cuda()[:, :, None, :]
    return h, q


def _same(a, b, what):
    for x, y, n in zip(a, b, ("out", "flags", "tokens")):
        assert torch.equal(x, y), f"{what}: {n} differs"


@pytest.mark.parametrize("v_group", [0, 32])
def test_device_count_matches_host_count(fkv, v_group):
    from foveated_kv_amd import synthetic

    B, Hq, Hkv, D, S, cap = 4, 32, 8, 128, 8192, 130
    _flush(f"device n_decode B={B} Hq={Hq} Hkv={Hkv} D={D} S={S} capacity={cap} v_group={v_group}")
    h, q = _layer(B, Hq, Hkv, D, S, seed=41, v_group=v_group)
    dk, dv = synthetic.make_decode(B, Hkv, cap, D, 41)
    dk, dv = torch.from_numpy(dk).cuda(), torch.from_numpy(dv).cuda()
    ndev = torch.zeros(1, dtype=torch.int32, device="cuda")
    for n in (0, 1, 63, 64, 65, 129, cap):
        ndev.fill_(n)
        got = h(q, dk, dv, n_decode=ndev)
        want = h(q, dk[:, :, :n].contiguous(), dv[:, :, :n].contiguous()) if n else h(q)
        torch.cuda.synchronize()
        _same(got, want, f"n={n}")
        if n:  # the first n rows of the capacity buffer, attended to in place (row stride = capacity)
            _same(h(q, dk[:, :, :n], dv[:, :, :n]), want, f"strided n={n}")
    # counts outside [0, capacity] are clamped by the kernel
    ndev.fill_(cap + 77)
    _same(h(q, dk, dv, n_decode=ndev), h(q, dk, dv), "n > capacity")
    ndev.fill_(-5)
    _same(h(q, dk, dv, n_decode=ndev), h(q), "n < 0")


def test_device_count_matches_host_count_turbo(fkv):
    """The same for a TurboQuant far tier (its own query staging)."""
    from foveated_kv_amd import ext, synthetic
    from foveated_kv_amd import turbo as tq

    B, Hq, Hkv, D, S, cap = 4, 32, 8, 128, 8192, 100
    _flush(f"device n_decode turbo B={B} Hq={Hq} Hkv={Hkv} D={D} S={S} capacity={cap}")
    k, v = synthetic.make_kv(B, Hkv, S, D, 45)
    cfg = ext.TierConfig()
    cfg.promo_headroom_min = 8
    cl = ext.CompressHandle(cfg).compress_layer(torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda(),
                                               with_archive=True)
    tc = tq.get_turbo_constants(D)
    tfar = tq.turbo_compress_keys(cl.archive_k, tc) + tq.turbo_compress_values(cl.archive_v)
    h = tq.TurboFoveatedHandle(cl.near_k, cl.near_v, *tfar, cl.near_valid, tc.Pi, tc.S, tc.centroids,
                               spike_margin=10.0)
    q = torch.from_numpy(synthetic.make_query(B, Hq, D, 45)).cuda()[:, :, None, :]
    dk, dv = synthetic.make_decode(B, Hkv, cap, D, 45)
    dk, dv = torch.from_numpy(dk).cuda(), torch.from_numpy(dv).cuda()
    ndev = torch.zeros(1, dtype=torch.int32, device="cuda")
    for n in (0, 1, 64, 65, cap):
        ndev.fill_(n)
        got = h(q, dk, dv, n_decode=ndev)
        want = h(q, dk[:, :, :n].contiguous(), dv[:, :, :n].contiguous()) if n else h(q)
        torch.cuda.synchronize()
        _same(got, want, f"turbo n={n}")


def test_device_count_rejects_bad_arguments(fkv):
    h, q = _layer(1, 8, 2, 64, 8192, seed=43)
    dk = torch.zeros((1, 2, 4, 64), dtype=torch.float16, device="cuda")
    with pytest.raises(TypeError):
        h(q, dk, dk, n_decode=torch.zeros(1, dtype=torch.int64, device="cuda"))
    with pytest.raises(ValueError):
        h(q, n_decode=torch.zeros(1, dtype=torch.int32, device="cuda"))


def test_graph_captured_decode_steps(fkv):
    """Append a row to the decode buffer and attend, captured once in a
    HIP graph, replayed step after step with eager work in between: every
    replay equals the eager host-count call on the same rows."""
    from foveated_kv_amd import synthetic

    B, Hq, Hkv, D, S, cap, steps = 4, 32, 8, 128, 8192, 96, 6
    _flush(f"graph decode steps B={B} Hq={Hq} Hkv={Hkv} D={D} S={S} capacity={cap} steps={steps}")
    h, q = _layer(B, Hq, Hkv, D, S, seed=47)
    rk, rv = synthetic.make_decode(B, Hkv, cap, D, 47)
    rk, rv = torch.from_numpy(rk).cuda(), torch.from_numpy(rv).cuda()
    first = 60  # rows already in the buffer when capture starts
    dk = torch.zeros((B, Hkv, cap, D), dtype=torch.float16, device="cuda")
    dv = torch.zeros_like(dk)
    dk[:, :, :first] = rk[:, :, :first]
    dv[:, :, :first] = rv[:, :, :first]
    ndev = torch.full((1,), first, dtype=torch.int32, device="cuda")
    new_k = torch.empty((B, Hkv, 1, D), dtype=torch.float16, device="cuda")
    new_v = torch.empty_like(new_k)
    qs = torch.empty_like(q)

    def step():
        pos = ndev.long()
        dk.index_copy_(2, pos, new_k)
        dv.index_copy_(2, pos, new_v)
        ndev.add_(1)
        return h(qs, dk, dv, n_decode=ndev)

    # eager warm-up allocates the handle's workspaces outside the capture
    new_k.copy_(rk[:, :, first:first + 1])
    new_v.copy_(rv[:, :, first:first + 1])
    qs.copy_(q)
    step()
    ndev.fill_(first)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        outs = step()
    torch.cuda.synchronize()
    ndev.fill_(first)
    gen = torch.Generator(device="cpu").manual_seed(5)
    for t in range(steps):
        n = first + t + 1
        new_k.copy_(rk[:, :, n - 1:n])
        new_v.copy_(rv[:, :, n - 1:n])
        qs.copy_(q + 0.25 * torch.randn(q.shape, generator=gen).to(q.device, q.dtype))
        g.replay()
        torch.cuda.synchronize()
        assert int(ndev.item()) == n
        want = h(qs, rk[:, :, :n].contiguous(), rv[:, :, :n].contiguous())
        torch.cuda.synchronize()
        _same([o.clone() for o in outs], want, f"replay {t} (n={n})")
        assert torch.equal(dk[:, :, :n], rk[:, :, :n])
        _flush(f"  replay {t}: n={n} equal")
