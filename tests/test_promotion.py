"""Promotion pipeline: the host drain filter against its restatement and
known answers (CPU), and the GPU side end to end (bit-exact rows, the
near_valid bump, attention after promotion)."""

import ctypes

import numpy as np
import pytest

from oracle import promotion as opromo

# ---------------------------------------------------------------------------
# helpers: the C-ABI drain on the host (no GPU work: borrowed archive rows)
# ---------------------------------------------------------------------------


class CDrain:
    def __init__(self, n_layers, cooldown=5, budget=8, spike_k=1):
        from foveated_kv_amd import _lib

        self.lib = _lib.load()
        self._lib = _lib
        self.h = ctypes.c_void_p()
        _lib.check(self.lib.fkv_promoter_create(n_layers, cooldown, budget, ctypes.byref(self.h)),
                   "fkv_promoter_create")
        _lib.check(self.lib.fkv_promoter_set_spike_k(self.h, spike_k), "fkv_promoter_set_spike_k")
        self.keep = []

    def archive(self, layer, k, v, idx):
        k = np.ascontiguousarray(k, np.float16)
        v = np.ascontiguousarray(v, np.float16)
        idx = np.ascontiguousarray(idx, np.int32)
        self.keep += [k, v, idx]
        B, H, S, D = k.shape
        self._lib.check(self.lib.fkv_promoter_register_archive(
            self.h, layer, k.ctypes.data_as(ctypes.c_void_p), v.ctypes.data_as(ctypes.c_void_p), B, H, S, D,
            idx.ctypes.data_as(ctypes.c_void_p), 0), "register_archive")

    def drain(self, layer, flags, tokens, far_idx, step):
        flags = np.ascontiguousarray(flags, np.int32)
        tokens = np.ascontiguousarray(tokens, np.int32)
        far_idx = np.ascontiguousarray(far_idx, np.int32)
        P = ctypes.c_void_p
        return self.lib.fkv_promoter_drain(self.h, layer, flags.ctypes.data_as(P), tokens.ctypes.data_as(P),
                                           far_idx.ctypes.data_as(P), flags.shape[0], flags.shape[1],
                                           far_idx.shape[1], far_idx.shape[2], step)

    def pending(self):
        n = self.lib.fkv_promoter_pending(self.h, None, 0)
        out = np.zeros((n, 4), np.int32)
        if n:
            self.lib.fkv_promoter_pending(self.h, out.ctypes.data_as(ctypes.c_void_p), n)
        return [tuple(int(x) for x in r) for r in out]

    def stats(self):
        c = self._lib.PromoterStatsC()
        self.lib.fkv_promoter_get_stats(self.h, ctypes.byref(c))
        return {f: int(getattr(c, f)) for f in self._lib.STATS_FIELDS}

    def __del__(self):
        if self.h.value:
            self.lib.fkv_promoter_destroy(self.h)


def _archive(Hkv, S, D, start=4, seed=0):
    rng = np.random.default_rng(seed)
    k = rng.standard_normal((1, Hkv, S, D)).astype(np.float16)
    v = rng.standard_normal((1, Hkv, S, D)).astype(np.float16)
    idx = np.broadcast_to(np.arange(start, start + S, dtype=np.int32), (Hkv, S)).copy()
    return k, v, idx


def _both(n_layers=2, cooldown=5, budget=8, spike_k=1):
    return CDrain(n_layers, cooldown, budget, spike_k), opromo.Pipeline(n_layers, cooldown, budget, spike_k)


def _register(c, o, layer, k, v, idx):
    c.archive(layer, k, v, idx)
    o.register_archive(layer, k, v, idx)


# ---------------------------------------------------------------------------
# known answers (each rule of promotion_pipeline.cpp:99-175), checked on both
# the restatement and the library
# ---------------------------------------------------------------------------

def test_gqa_dedup_keeps_first_flagged_query_head():
    c, o = _both()
    Hq, Hkv, S = 8, 2, 40
    k, v, idx = _archive(Hkv, S, 4)
    _register(c, o, 0, k, v, idx)
    far_idx = idx[None]
    flags = np.zeros((1, Hq), np.int32)
    tokens = np.zeros((1, Hq), np.int32)
    flags[0, [1, 2, 5]] = 1          # heads 1, 2 -> kv 0; head 5 -> kv 1
    tokens[0, 1], tokens[0, 2], tokens[0, 5] = 7, 9, 3
    for impl in (c, o):
        assert impl.drain(0, flags, tokens, far_idx, 0) == 2
    assert c.pending() == [(0, 0, 7, 11), (0, 1, 3, 7)] == o.queue
    assert c.stats()["spikes_detected"] == o.stats["spikes_detected"] == 2


def test_cooldown_and_position_dedup():
    c, o = _both(cooldown=5)
    k, v, idx = _archive(1, 30, 4)
    _register(c, o, 0, k, v, idx)
    far_idx = idx[None]
    f = np.ones((1, 1), np.int32)
    for step, tok in [(0, 5), (3, 6), (5, 5), (11, 6)]:
        for impl in (c, o):
            impl.drain(0, f, np.full((1, 1), tok, np.int32), far_idx, step)
    # step 0 queues 5; step 3 is cooled down; step 5 finds 5 already promoted;
    # step 11 queues 6
    assert [r[2] for r in c.pending()] == [5, 6] == [r[2] for r in o.queue]
    s = c.stats()
    assert s == o.stats
    assert (s["spikes_detected"], s["spikes_cooled_down"], s["spikes_deduplicated"], s["spikes_queued"]) == (4, 1, 1, 2)


def test_budget_out_of_range_and_missing_rows():
    c, o = _both(budget=2)
    Hkv, S = 4, 20
    k, v, idx = _archive(Hkv, S, 4)
    idx[2, 3] = 999                      # head 2, far row 3 is not in the archive under its far position
    _register(c, o, 0, k, v, idx)
    far_idx = np.broadcast_to(np.arange(4, 4 + S, dtype=np.int32), (1, Hkv, S)).copy()
    flags = np.ones((1, Hkv), np.int32)
    tokens = np.array([[-1, S, 3, 1]], np.int32)   # out of range twice, then a missing row, then ok
    for impl in (c, o):
        assert impl.drain(0, flags, tokens, far_idx, 0) == 1
    assert c.pending() == o.queue == [(0, 3, 1, 5)]
    s = c.stats()
    assert s == o.stats and s["spikes_detected"] == 4 and s["spikes_queued"] == 1
    # a layer without an archive and an invalid layer queue nothing
    for impl in (c, o):
        assert impl.drain(1, flags, tokens, far_idx, 0) == 0
        assert impl.drain(7, flags, tokens, far_idx, 0) == 0


def test_drain_matches_restatement_on_random_streams():
    rng = np.random.default_rng(5)
    c, o = _both(n_layers=3, cooldown=3, budget=5)
    B, Hq, Hkv, S = 2, 16, 4, 50
    for layer in range(3):
        k, v, idx = _archive(Hkv, S, 10, seed=layer)
        _register(c, o, layer, k, v, idx)
    far_idx = np.broadcast_to(np.arange(10, 10 + S, dtype=np.int32), (B, Hkv, S)).copy()
    for step in range(40):
        for layer in range(3):
            flags = (rng.random((B, Hq)) < 0.3).astype(np.int32)
            tokens = rng.integers(-2, S + 2, size=(B, Hq)).astype(np.int32)
            assert c.drain(layer, flags, tokens, far_idx, step) == o.drain(layer, flags, tokens, far_idx, step)
    assert c.pending() == o.queue
    assert c.stats() == o.stats
    assert o.stats["spikes_cooled_down"] > 0 and o.stats["spikes_deduplicated"] > 0


# ---------------------------------------------------------------------------
# several spiking tokens per query head (spike_k > 1: the benchmark's "up to
# 32 far tokens per head per step"; flags are counts, tokens (B, Hq, K))
# ---------------------------------------------------------------------------

def test_spike_k_known_answers():
    c, o = _both(n_layers=1, cooldown=2, budget=6, spike_k=4)
    Hq, Hkv, S = 4, 2, 40
    k, v, idx = _archive(Hkv, S, 4)
    _register(c, o, 0, k, v, idx)
    far_idx = idx[None]
    flags = np.array([[0, 3, 2, 4]], np.int32)            # kv 0: head 1 (3 tokens); kv 1: head 2 wins over 3
    tokens = np.full((1, Hq, 4), -1, np.int32)
    tokens[0, 1, :3] = [7, 9, 11]
    tokens[0, 2, :2] = [5, 5 + 0]                          # a repeated token: the second is a duplicate
    tokens[0, 3] = [1, 2, 3, 4]
    for impl in (c, o):
        assert impl.drain(0, flags, tokens, far_idx, 0) == 4
    assert c.pending() == o.queue == [(0, 0, 7, 11), (0, 0, 9, 13), (0, 0, 11, 15), (0, 1, 5, 9)]
    s = c.stats()
    assert s == o.stats
    assert (s["spikes_detected"], s["spikes_queued"], s["spikes_deduplicated"]) == (2, 4, 1)
    # step 1: both heads cooled down (once per head, not per token)
    for impl in (c, o):
        assert impl.drain(0, flags, tokens, far_idx, 1) == 0
    assert c.stats()["spikes_cooled_down"] == o.stats["spikes_cooled_down"] == 2
    # step 2: head 0 queues 4, head 1 the 2 tokens the budget (6) leaves
    flags2 = np.array([[4, 4, 4, 4]], np.int32)
    tokens2 = np.zeros((1, Hq, 4), np.int32)
    tokens2[0, 0] = [20, 21, 22, 23]
    tokens2[0, 2] = [30, 31, 32, 33]
    for impl in (c, o):
        assert impl.drain(0, flags2, tokens2, far_idx, 2) == 6
    assert [r[3] for r in o.queue[-6:]] == [24, 25, 26, 27, 34, 35]
    # step 5: head 1's first token is now a duplicate; the budget then
    # stops it after two more
    tokens2[0, 0] = [24, 25, 26, 27]
    tokens2[0, 2] = [30, 34, 35, 36]
    for impl in (c, o):
        assert impl.drain(0, flags2, tokens2, far_idx, 5) == 6
    assert [r[3] for r in o.queue[-6:]] == [28, 29, 30, 31, 38, 39]
    assert c.pending() == o.queue
    s = c.stats()
    assert s == o.stats and s["spikes_deduplicated"] == 2


def test_spike_k_counts_above_k_are_clamped_and_k1_ignores_counts():
    c, o = _both(n_layers=1, cooldown=0, budget=100, spike_k=2)
    k, v, idx = _archive(1, 30, 4)
    _register(c, o, 0, k, v, idx)
    tokens = np.array([[[3, 4]]], np.int32)
    for impl in (c, o):
        assert impl.drain(0, np.array([[9]], np.int32), tokens, idx[None], 0) == 2
    assert c.pending() == o.queue
    c1, o1 = _both(n_layers=1, cooldown=0, budget=100)
    _register(c1, o1, 0, k, v, idx)
    for impl in (c1, o1):   # spike_k = 1: any nonzero flag is one token, as the reference
        assert impl.drain(0, np.array([[5]], np.int32), np.array([[3]], np.int32), idx[None], 0) == 1


@pytest.mark.parametrize("K", [2, 5, 32])
def test_spike_k_drain_matches_restatement_on_random_streams(K):
    rng = np.random.default_rng(K)
    c, o = _both(n_layers=2, cooldown=2, budget=3 * K, spike_k=K)
    B, Hq, Hkv, S = 2, 16, 4, 80
    for layer in range(2):
        k, v, idx = _archive(Hkv, S, 10, seed=layer)
        _register(c, o, layer, k, v, idx)
    far_idx = np.broadcast_to(np.arange(10, 10 + S, dtype=np.int32), (B, Hkv, S)).copy()
    for step in range(30):
        for layer in range(2):
            flags = np.where(rng.random((B, Hq)) < 0.3, rng.integers(1, K + 3, size=(B, Hq)), 0).astype(np.int32)
            tokens = np.stack([rng.permutation(S)[:K] for _ in range(B * Hq)]).reshape(B, Hq, K).astype(np.int32)
            tokens[rng.random((B, Hq, K)) < 0.05] = -1
            assert c.drain(layer, flags, tokens, far_idx, step) == o.drain(layer, flags, tokens, far_idx, step)
    assert c.pending() == o.queue
    assert c.stats() == o.stats
    assert o.stats["spikes_deduplicated"] > 0 and o.stats["spikes_cooled_down"] > 0


def test_spike_k_range_is_checked():
    from foveated_kv_amd import _lib

    lib = _lib.load()
    c = CDrain(1)
    for bad in (0, 33, -1):
        assert lib.fkv_promoter_set_spike_k(c.h, bad) == _lib.FKV_EINVAL


# ---------------------------------------------------------------------------
# GPU side
# ---------------------------------------------------------------------------

def _layer(B, Hkv, D, S, seed, headroom_min=8):
    import torch

    from foveated_kv_amd import ext, synthetic

    k, v = synthetic.make_kv(B, Hkv, S, D, seed)
    cfg = ext.TierConfig()
    cfg.promo_headroom_min = headroom_min
    cfg.promo_headroom_pct = 0.5
    cl = ext.CompressHandle(cfg).compress_layer(torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda())
    h = ext.FoveatedHandle(cl.near_k, cl.near_v, cl.far_k, cl.far_v, cl.far_v_scale, cl.far_v_zero, cl.near_valid,
                           spike_margin=10.0)
    return k, v, cl, h


@pytest.mark.gpu
@pytest.mark.parametrize("arc", ["pinned", "device"])
@pytest.mark.parametrize("B", [1, 2])
def test_promotion_rows_bit_exact_and_near_valid(orc, B, arc):
    """The host drain + flush against the CPU restatement: promoted rows
    bit-exact, near_valid and statistics equal, with the archive in pinned
    host memory (the reference's placement) or in device memory (rows
    copied device to device)."""
    import torch

    from foveated_kv_amd.promotion import PromotionPipeline
    from foveated_kv_amd.tier_cache import TierConfig, tier_index_tensors

    Hkv, Hq, D, S = 2, 8, 128, 1000
    print(f"promotion B={B} Hkv={Hkv} D={D} S={S} archive={arc}", flush=True)
    k, v, cl, h = _layer(B, Hkv, D, S, 31)
    tb = TierConfig(promo_headroom_min=8).tier_boundaries(S)
    _, far_idx = tier_index_tensors(tb, S, B, Hkv, "cpu")
    far_idx = far_idx.numpy()
    pipe = PromotionPipeline(1, cooldown_steps=0, max_per_drain=8)
    pipe.register_archive_tensors(0, cl.archive_k, cl.archive_v, far_idx, device=arc == "device")
    pipe.register_blob(0, h.get_blob_info())
    ref = opromo.Pipeline(1, 0, 8)
    ref.register_archive(0, cl.archive_k.cpu().numpy(), cl.archive_v.cpu().numpy(), far_idx[0])
    near_k = {0: cl.near_k.cpu().numpy().copy()}
    near_v = {0: cl.near_v.cpu().numpy().copy()}
    nv = {0: cl.near_valid.cpu().numpy().copy()}
    rng = np.random.default_rng(3)
    for step in range(6):
        flags = np.ones((B, Hq), np.int32)
        tokens = rng.integers(0, far_idx.shape[2], size=(B, Hq)).astype(np.int32)
        pipe.drain_spikes(0, torch.from_numpy(flags), torch.from_numpy(tokens), far_idx, step)
        ref.drain(0, flags, tokens, far_idx, step)
        ref.commit(near_k, near_v, nv, {0: cl.near_k.shape[2]})
    pipe.order(0)
    torch.cuda.synchronize()
    gk, gv = h.export_near()
    assert h.read_near_valid() == [int(x) for x in nv[0]] == pipe.near_valid(0)
    assert np.array_equal(gk.cpu().numpy().view(np.uint16), near_k[0].view(np.uint16))
    assert np.array_equal(gv.cpu().numpy().view(np.uint16), near_v[0].view(np.uint16))
    assert pipe.get_stats() == ref.stats and ref.stats["promotions_completed"] > 0
    # the kernel attends to the promoted rows: parity with the oracle on the exported tier
    q = torch.from_numpy(np.random.default_rng(4).standard_normal((B, Hq, D)).astype(np.float16)).cuda()
    out, flags_o, tokens_o = h(q[:, :, None])
    torch.cuda.synchronize()
    o, _, _, _, _ = orc.attend_kernel(q.cpu().numpy(), near_k[0], near_v[0], nv[0], cl.far_k.cpu().numpy(),
                                      cl.far_v.cpu().numpy(), cl.far_v_scale.cpu().numpy(),
                                      cl.far_v_zero.cpu().numpy(), spike_margin=10.0)
    got = out[:, :, 0].float().cpu().numpy()
    assert np.abs(got - o).max() <= 2e-3 and orc.cosine(got, o) >= 0.9999


@pytest.mark.gpu
def test_promotion_headroom_full_is_counted():
    import torch

    from foveated_kv_amd.promotion import PromotionPipeline
    from foveated_kv_amd.tier_cache import TierConfig, tier_index_tensors

    B, Hkv, Hq, D, S = 1, 1, 4, 64, 100   # R = 36, headroom = 18
    _, _, cl, h = _layer(B, Hkv, D, S, 32, headroom_min=2)
    tb = TierConfig(promo_headroom_min=2).tier_boundaries(S)
    _, far_idx = tier_index_tensors(tb, S, B, Hkv, "cpu")
    far_idx = far_idx.numpy()
    cap = cl.near_k.shape[2]
    pipe = PromotionPipeline(1, cooldown_steps=0, max_per_drain=8)
    pipe.register_archive_tensors(0, cl.archive_k, cl.archive_v, far_idx)
    pipe.register_blob(0, h)
    n_far = far_idx.shape[2]
    for step in range(n_far):
        pipe.drain_spikes(0, np.ones((1, Hq), np.int32), np.full((1, Hq), step, np.int32), far_idx, step)
    pipe.synchronize()
    s = pipe.get_stats()
    assert h.read_near_valid() == [cap]
    assert s["promotions_completed"] == cap - tb["R_actual"]
    assert s["promotions_headroom_full"] == n_far - s["promotions_completed"]


@pytest.mark.gpu
def test_promotion_from_archive_files(tmp_path):
    """The reference's on-disk archive format (disk_archive.py:127-185):
    (H_kv, S_arc, D) fp16 raw per layer, batch 0."""
    import torch

    from foveated_kv_amd.promotion import PromotionPipeline
    from foveated_kv_amd.tier_cache import TierConfig, tier_index_tensors

    B, Hkv, D, S = 1, 2, 64, 512
    _, _, cl, h = _layer(B, Hkv, D, S, 33)
    tb = TierConfig(promo_headroom_min=8).tier_boundaries(S)
    _, far_idx = tier_index_tensors(tb, S, B, Hkv, "cpu")
    far_idx = far_idx.numpy()
    ak = cl.archive_k[0].cpu().numpy()
    av = cl.archive_v[0].cpu().numpy()
    pk, pv = tmp_path / "archive_k_layer0.bin", tmp_path / "archive_v_layer0.bin"
    ak.tofile(pk)
    av.tofile(pv)
    pipe = PromotionPipeline(1, cooldown_steps=0)
    pipe.register_blob(0, h)
    # an unreadable archive leaves the layer without one: drains queue nothing
    assert not pipe.register_archive(0, tmp_path / "missing.bin", pv, Hkv, ak.shape[1], D, far_idx[0])
    assert pipe.drain_spikes(0, np.ones((1, 8), np.int32), np.zeros((1, 8), np.int32), far_idx, 0) == 0
    assert pipe.register_archive(0, pk, pv, Hkv, ak.shape[1], D, far_idx[0])
    r0 = h.read_near_valid()
    tokens = np.array([[10, 10, 10, 10, 20, 20, 20, 20]], np.int32)
    pipe.drain_spikes(0, np.ones((1, 8), np.int32), tokens, far_idx, 1)
    pipe.order(0)
    torch.cuda.synchronize()
    gk, gv = h.export_near()
    nv = h.read_near_valid()
    assert nv == [r0[0] + 1, r0[1] + 1]
    for hh, tok in ((0, 10), (1, 20)):
        assert np.array_equal(gk[0, hh, r0[hh]].cpu().numpy().view(np.uint16), ak[hh, tok].view(np.uint16))
        assert np.array_equal(gv[0, hh, r0[hh]].cpu().numpy().view(np.uint16), av[hh, tok].view(np.uint16))


@pytest.mark.gpu
@pytest.mark.parametrize("B,cooldown,budget,headroom_min,arc", [(1, 0, 8, 8, "pinned"), (2, 3, 2, 8, "pinned"),
                                                                (1, 1, 8, 2, "pinned"), (3, 2, 3, 8, "pinned"),
                                                                (1, 0, 8, 8, "device"), (3, 2, 3, 8, "device")])
def test_device_drain_matches_host_restatement(orc, B, cooldown, budget, headroom_min, arc):
    """drain_spikes_device (filter + promotion in one kernel, spike outputs
    and far_idx in device memory) against the CPU restatement of the host
    drain + flush on random flag streams: same near tiers, near_valid and
    statistics.  Batches above 1 keep the step on the device and let the
    drain advance it.  The archive rows come from pinned host memory or,
    registered with device=True, from device memory."""
    import torch

    from foveated_kv_amd.promotion import PromotionPipeline
    from foveated_kv_amd.tier_cache import TierConfig, tier_index_tensors

    Hkv, Hq, D, S = 4, 16, 128, 900
    print(f"device drain B={B} cooldown={cooldown} budget={budget} headroom_min={headroom_min} archive={arc}",
          flush=True)
    k, v, cl, h = _layer(B, Hkv, D, S, 41, headroom_min=headroom_min)
    tb = TierConfig(promo_headroom_min=headroom_min).tier_boundaries(S)
    _, far_idx = tier_index_tensors(tb, S, B, Hkv, "cpu")
    far_idx = far_idx.numpy()
    fdev = torch.from_numpy(far_idx).cuda().contiguous()
    pipe = PromotionPipeline(1, cooldown_steps=cooldown, max_per_drain=budget)
    pipe.register_archive_tensors(0, cl.archive_k, cl.archive_v, far_idx, device=arc == "device")
    pipe.register_blob(0, h)
    ref = opromo.Pipeline(1, cooldown, budget)
    ref.register_archive(0, cl.archive_k.cpu().numpy(), cl.archive_v.cpu().numpy(), far_idx[0])
    near_k = {0: cl.near_k.cpu().numpy().copy()}
    near_v = {0: cl.near_v.cpu().numpy().copy()}
    nv = {0: cl.near_valid.cpu().numpy().copy()}
    rng = np.random.default_rng(B * 10 + budget)
    n_far = far_idx.shape[2]
    step_d = torch.zeros(1, dtype=torch.int32, device="cuda") if B > 1 else None
    for step in range(30):
        flags = (rng.random((B, Hq)) < 0.4).astype(np.int32)
        tokens = rng.integers(0, min(n_far, 40), size=(B, Hq)).astype(np.int32)  # repeats exercise dedup
        tokens[rng.random((B, Hq)) < 0.05] = -1
        fl, tk = torch.from_numpy(flags).cuda(), torch.from_numpy(tokens).cuda()
        if step_d is None:
            pipe.drain_spikes_device(0, fl, tk, fdev, step)
        else:
            pipe.drain_spikes_device(0, fl, tk, fdev, step_d, advance_step=True)
        ref.drain(0, flags, tokens, far_idx, step)
        ref.commit(near_k, near_v, nv, {0: cl.near_k.shape[2]})
    torch.cuda.synchronize()
    if step_d is not None:
        assert int(step_d.item()) == 30
    gk, gv = h.export_near()
    assert h.read_near_valid() == [int(x) for x in nv[0]]
    assert np.array_equal(gk.cpu().numpy().view(np.uint16), near_k[0].view(np.uint16))
    assert np.array_equal(gv.cpu().numpy().view(np.uint16), near_v[0].view(np.uint16))
    assert pipe.get_stats() == ref.stats and ref.stats["promotions_completed"] > 0


@pytest.mark.gpu
@pytest.mark.parametrize("B,K,cooldown,budget,arc", [(1, 4, 0, 8, "pinned"), (2, 32, 2, 40, "pinned"),
                                                     (1, 32, 1, 5, "pinned"), (2, 6, 3, 64, "pinned"),
                                                     (2, 32, 2, 40, "device")])
def test_device_drain_top_k_matches_host_restatement(orc, B, K, cooldown, budget, arc):
    """The device drain with spike_k = K > 1 (each KV head's first flagged
    query head hands up to K tokens through the filter, the budget checked
    before each token) against the CPU restatement on random streams: spike
    counts 0..K+2 (clamped to K), token lists with repeated positions and -1
    entries, budgets that stop a head's list part way.  Same near tiers,
    near_valid and statistics."""
    import torch

    from foveated_kv_amd.promotion import PromotionPipeline
    from foveated_kv_amd.tier_cache import TierConfig, tier_index_tensors

    Hkv, Hq, D, S = 4, 16, 128, 1200
    print(f"device drain top-K B={B} K={K} cooldown={cooldown} budget={budget}", flush=True)
    k, v, cl, h = _layer(B, Hkv, D, S, 43, headroom_min=48)
    tb = TierConfig(promo_headroom_min=48).tier_boundaries(S)
    _, far_idx = tier_index_tensors(tb, S, B, Hkv, "cpu")
    far_idx = far_idx.numpy()
    fdev = torch.from_numpy(far_idx).cuda().contiguous()
    pipe = PromotionPipeline(1, cooldown_steps=cooldown, max_per_drain=budget, spike_k=K)
    pipe.register_archive_tensors(0, cl.archive_k, cl.archive_v, far_idx, device=arc == "device")
    pipe.register_blob(0, h)
    ref = opromo.Pipeline(1, cooldown, budget, K)
    ref.register_archive(0, cl.archive_k.cpu().numpy(), cl.archive_v.cpu().numpy(), far_idx[0])
    near_k = {0: cl.near_k.cpu().numpy().copy()}
    near_v = {0: cl.near_v.cpu().numpy().copy()}
    nv = {0: cl.near_valid.cpu().numpy().copy()}
    rng = np.random.default_rng(B * 100 + K + budget)
    n_far = far_idx.shape[2]
    for step in range(24):
        flags = np.where(rng.random((B, Hq)) < 0.4, rng.integers(1, K + 3, size=(B, Hq)), 0).astype(np.int32)
        tokens = rng.integers(0, min(n_far, 3 * K + 20), size=(B, Hq, K)).astype(np.int32)  # repeats
        tokens[rng.random((B, Hq, K)) < 0.05] = -1
        fl, tk = torch.from_numpy(flags).cuda(), torch.from_numpy(tokens).cuda()
        pipe.drain_spikes_device(0, fl, tk, fdev, step)
        ref.drain(0, flags, tokens, far_idx, step)
        ref.commit(near_k, near_v, nv, {0: cl.near_k.shape[2]})
    torch.cuda.synchronize()
    gk, gv = h.export_near()
    assert h.read_near_valid() == [int(x) for x in nv[0]]
    assert np.array_equal(gk.cpu().numpy().view(np.uint16), near_k[0].view(np.uint16))
    assert np.array_equal(gv.cpu().numpy().view(np.uint16), near_v[0].view(np.uint16))
    assert pipe.get_stats() == ref.stats and ref.stats["promotions_completed"] > 0
    assert ref.stats["spikes_deduplicated"] > 0


@pytest.mark.gpu
def test_device_archive_rejects_host_rows():
    """register_archive_tensors(device=True) takes GPU tensors only, and the
    C entry point refuses rows that are not in device memory."""
    import torch

    from foveated_kv_amd.promotion import PromotionPipeline

    pipe = PromotionPipeline(1)
    k = torch.zeros((1, 2, 10, 64), dtype=torch.float16)
    idx = np.arange(20, dtype=np.int32).reshape(2, 10)
    with pytest.raises(ValueError):
        pipe.register_archive_tensors(0, k, k, idx, device=True)
    rc = pipe._lib.fkv_promoter_register_archive_device(pipe._h, 0, ctypes.c_void_p(k.data_ptr()),
                                                        ctypes.c_void_p(k.data_ptr()), 1, 2, 10, 64,
                                                        idx.ctypes.data_as(ctypes.c_void_p))
    assert rc != 0
    kd = k.cuda()
    assert pipe._lib.fkv_promoter_register_archive_device(pipe._h, 0, ctypes.c_void_p(kd.data_ptr()),
                                                          ctypes.c_void_p(kd.data_ptr()), 1, 2, 10, 64,
                                                          idx.ctypes.data_as(ctypes.c_void_p)) == 0


@pytest.mark.gpu
def test_device_drain_step_advance_without_work():
    """advance_step advances the device step on every successful call, also
    where the drain has nothing to launch (a layer with no archive or blob
    registered); it needs a device step (TypeError in Python, FKV_EINVAL
    through the C ABI)."""
    import ctypes

    import torch

    from foveated_kv_amd import _lib
    from foveated_kv_amd.promotion import PromotionPipeline
    from foveated_kv_amd.tier_cache import TierConfig, tier_index_tensors

    print("device drain step advance", flush=True)
    B, Hkv, D, S = 1, 2, 64, 400
    k, v, cl, h = _layer(B, Hkv, D, S, 7)
    _, far_idx = tier_index_tensors(TierConfig(promo_headroom_min=8).tier_boundaries(S), S, B, Hkv, "cpu")
    far_idx = far_idx.numpy()
    pipe = PromotionPipeline(2, cooldown_steps=1, max_per_drain=4)
    pipe.register_archive_tensors(0, cl.archive_k, cl.archive_v, far_idx)
    pipe.register_blob(0, h)
    fdev = torch.from_numpy(far_idx).cuda().contiguous()
    flags = torch.zeros((B, 4 * Hkv), dtype=torch.int32, device="cuda")
    toks = torch.full((B, 4 * Hkv), -1, dtype=torch.int32, device="cuda")
    step_d = torch.full((1,), 5, dtype=torch.int32, device="cuda")
    pipe.drain_spikes_device(0, flags, toks, fdev, step_d, advance_step=True)  # the drain kernel
    pipe.drain_spikes_device(1, flags, toks, fdev, step_d, advance_step=True)  # nothing registered
    pipe.drain_spikes_device(0, flags, toks, fdev, step_d)  # read only
    torch.cuda.synchronize()
    assert int(step_d.item()) == 7
    with pytest.raises(TypeError):
        pipe.drain_spikes_device(0, flags, toks, fdev, 3, advance_step=True)
    lib = _lib.load()
    rc = lib.fkv_promoter_drain_device(pipe._h, 0, _lib.ptr(flags), _lib.ptr(toks), _lib.ptr(fdev), B, 4 * Hkv,
                                       Hkv, fdev.shape[2], 0, None, 1, _lib.stream_ptr(flags.device))
    assert rc == _lib.FKV_EINVAL
    torch.cuda.synchronize()
    assert int(step_d.item()) == 7
