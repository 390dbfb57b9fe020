"""End-to-end compress + decode + promote loop (the C5 workload, at reduced
shapes and at its full shape) on the GPU: importance partition, a growing
decode buffer, per-step query drift that triggers spikes, and promotion of
exact fp16 rows into the near headroom.  The output and spike fields of
every step (every 16th at the full shape) are checked against the oracle
run on the state the CPU restatement of the promotion pipeline tracks; the
final near tier is bit-exact."""

import numpy as np
import pytest
import torch

from oracle import promotion as opromo

pytestmark = pytest.mark.gpu


def _np(t):
    return t.detach().cpu().numpy()


@pytest.mark.parametrize("B,Hq,Hkv,D,S,steps,vg,mode", [(1, 16, 4, 128, 8192, 24, 0, "host"),
                                                        (1, 14, 2, 64, 2048, 16, 32, "host"),
                                                        (1, 16, 4, 128, 8192, 24, 0, "device"),
                                                        (2, 16, 2, 64, 3000, 20, 32, "device"),
                                                        (1, 16, 4, 128, 8192, 24, 0, "graph"),
                                                        (2, 16, 2, 64, 3000, 20, 32, "graph")])
def test_decode_promote_loop_matches_oracle_every_step(orc, B, Hq, Hkv, D, S, steps, vg, mode):
    """mode: "host" drains the read-back spike outputs on the host; "device"
    drains with the device kernel; "graph" captures step 1's attention (decode
    count on the device) and device drain (step on the device) in a HIP graph
    and replays it for every later step."""
    _loop(orc, B, Hq, Hkv, D, S, steps, vg, mode, check_every=1)


def test_c5_full_loop(orc):
    """C5 at its full shape, as the benchmark runs it: Hq=64, Hkv=8, D=128,
    64K context, B=1, importance partition, 128 decode steps captured in one
    HIP graph (device decode count, device drain).  The spike outputs of
    every step drive the CPU restatement of the promotion pipeline; the
    attention output and spikes are checked against the oracle every 16th
    step and at the last; the final near tier, near_valid and statistics are
    bit-exact."""
    _loop(orc, 1, 64, 8, 128, 65536, 128, 0, "graph", check_every=16)


def test_c5_full_loop_top32(orc):
    """C5 with its stated promotion rule, "up to 32 far tokens per head per
    step (cooldown + GQA dedup)": spike_k = 32, a budget of 32 tokens per KV
    head (256 per step), the rest as test_c5_full_loop.  The spike counts and
    token lists of the checked steps match the oracle's top-32 of the exact
    far scores (ties within rounding); the final near tier, near_valid and
    statistics are bit-exact against the restated drain fed the GPU's own
    spike outputs."""
    _loop(orc, 1, 64, 8, 128, 65536, 128, 0, "graph", check_every=16, spike_k=32, budget=256)


@pytest.mark.parametrize("mode", ["host", "device"])
def test_decode_promote_loop_top_k(orc, mode):
    """Several spiking tokens per head per step (spike_k = 6, budget 12)
    through the host drain and the device drain, every step checked."""
    _loop(orc, 2, 16, 4, 128, 6000, 20, 0, mode, check_every=1, spike_k=6, budget=12)


def _loop(orc, B, Hq, Hkv, D, S, steps, vg, mode, check_every, spike_k=1, budget=8):
    from foveated_kv_amd import ext, synthetic
    from foveated_kv_amd.promotion import PromotionPipeline

    from _parity import check_topk, record

    seed = S + steps
    case = f"e2e B={B} Hq={Hq} Hkv={Hkv} D={D} S={S} steps={steps} v_group={vg} mode={mode} spike_k={spike_k}"
    print(case, flush=True)
    worst_err, worst_cos, checked = 0.0, 1.0, 0
    k, v = synthetic.make_kv(B, Hkv, S, D, seed)
    q0 = synthetic.make_query(B, Hq, D, seed)
    imp = torch.from_numpy(synthetic.make_importance(B, Hkv, S, seed)).cuda()
    cfg = ext.TierConfig()
    cfg.promo_headroom_min = 8
    cfg.v_group = vg
    _, far_idx = ext.partition_importance(cfg, imp, B, Hkv, S)
    far_idx = _np(far_idx)
    synthetic.inject_spikes_at(k, q0, far_idx, 0.02, seed)
    cl = ext.CompressHandle(cfg).compress_layer(torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda(),
                                                importance=imp)
    assert np.array_equal(_np(cl.far_idx), far_idx)
    h = ext.FoveatedHandle(cl.near_k, cl.near_v, cl.far_k, cl.far_v, cl.far_v_scale, cl.far_v_zero,
                           cl.near_valid, spike_margin=10.0, spike_k=spike_k)
    pipe = PromotionPipeline(1, cooldown_steps=5, max_per_drain=budget, spike_k=spike_k)
    pipe.register_archive_tensors(0, cl.archive_k, cl.archive_v, far_idx)
    pipe.register_blob(0, h)
    ref = opromo.Pipeline(1, 5, budget, spike_k)
    ref.register_archive(0, _np(cl.archive_k), _np(cl.archive_v), far_idx[0])
    near_k, near_v, nv = {0: _np(cl.near_k).copy()}, {0: _np(cl.near_v).copy()}, {0: _np(cl.near_valid).copy()}
    far = [_np(getattr(cl, n)) for n in ("far_k", "far_v", "far_v_scale", "far_v_zero")]
    fdev = cl.far_idx.to(torch.int32).contiguous()
    qs = synthetic.drift_queries(q0, steps, 0.05, seed)
    dk, dv = synthetic.make_decode(B, Hkv, steps, D, seed)
    dkt, dvt = torch.from_numpy(dk).cuda(), torch.from_numpy(dv).cuda()
    lut = orc.decode_fp8(np.arange(256, dtype=np.uint8)).astype(np.float64)
    flagged = 0
    q_st = torch.empty((B, Hq, 1, D), dtype=torch.float16, device="cuda")
    step_d = torch.zeros(1, dtype=torch.int32, device="cuda")
    n_d = torch.zeros(1, dtype=torch.int32, device="cuda")
    graph = graph_res = None

    def one():  # the captured step: count from the step, attention, drain (which advances the step)
        torch.add(step_d, 1, out=n_d)
        res = h(q_st, dkt, dvt, n_decode=n_d)
        pipe.drain_spikes_device(0, res[1], res[2], fdev, step_d, advance_step=True)
        return res

    for t in range(steps):
        if mode == "host":
            pipe.order(0)
        q = torch.from_numpy(qs[t]).cuda()
        n = t + 1
        if mode == "graph":
            q_st.copy_(q[:, :, None])
            if t == 0:
                out, flags, toks = one()  # eager: sizes the workspaces before capture
            else:
                if graph is None:
                    torch.cuda.synchronize()
                    graph = torch.cuda.CUDAGraph()
                    with torch.cuda.graph(graph):
                        graph_res = one()
                graph.replay()
                out, flags, toks = graph_res
        else:
            out, flags, toks = h(q[:, :, None], dkt[:, :, :n].contiguous(), dvt[:, :, :n].contiguous())
        torch.cuda.synchronize()
        if mode == "graph":
            assert int(step_d.item()) == n
        fl, tk = _np(flags), _np(toks)
        if t % check_every == 0 or t == steps - 1:
            o, kf, kt, mf, mn, fsc = orc.attend_kernel(qs[t], near_k[0], near_v[0], nv[0], *far, dk[:, :, :n],
                                                       dv[:, :, :n], spike_margin=10.0, return_far_scores=True)
            got = _np(out)[:, :, 0].astype(np.float64)
            err, cos = np.abs(got - o).max(), orc.cosine(got, o)
            assert err <= 2e-3 and cos >= 0.9999, (t, err, cos)
            worst_err, worst_cos, checked = max(worst_err, err), min(worst_cos, cos), checked + 1
            if spike_k > 1:
                for b in range(B):
                    for hq in range(Hq):
                        check_topk(fsc[b, hq], mn[b, hq] + 10.0, spike_k, int(fl[b, hq]), tk[b, hq])
        if spike_k > 1:
            flagged += int((fl > 0).sum())
        elif t % check_every == 0 or t == steps - 1:
            for b, hq in np.argwhere(fl != kf):
                assert abs(mf[b, hq] - mn[b, hq] - 10.0) < 1e-4, (t, b, hq)
            for b, hq in np.argwhere(tk != kt):  # only on a near tie of the exact far scores
                qs32 = qs[t][b, hq].astype(np.float32) * np.float32(1 / np.sqrt(np.float32(D)))
                sc = lut[far[0][b, hq // (Hq // Hkv)]] @ qs32.astype(np.float64)
                assert abs(sc[tk[b, hq]] - sc[kt[b, hq]]) <= 1e-5 * (1 + abs(sc.max())), (t, b, hq)
        if spike_k == 1:
            flagged += int(fl.sum())
        # both pipelines see the GPU's spike outputs, so their states stay comparable
        if mode == "device":
            pipe.drain_spikes_device(0, flags, toks, fdev, t)
        elif mode == "host":
            pipe.drain_spikes(0, flags, toks, far_idx, t)
        ref.drain(0, fl, tk, far_idx, t)
        ref.commit(near_k, near_v, nv, {0: cl.near_k.shape[2]})
    pipe.synchronize()
    gk, gv = h.export_near()
    assert flagged > 0 and ref.stats["promotions_completed"] > 0
    assert h.read_near_valid() == [int(x) for x in nv[0]]
    assert np.array_equal(_np(gk).view(np.uint16), near_k[0].view(np.uint16))
    assert np.array_equal(_np(gv).view(np.uint16), near_v[0].view(np.uint16))
    assert pipe.get_stats() == ref.stats
    record(f"{case} (checked {checked} steps)", maxabs_kernel=worst_err, cos_kernel=worst_cos, flagged=flagged,
           promotions=ref.stats["promotions_completed"])
    print(f"  promotions {ref.stats['promotions_completed']} over {steps} steps, stats {ref.stats}", flush=True)
    if spike_k > 1:  # more than one row per head in some drain
        assert ref.stats["promotions_completed"] > ref.stats["spikes_detected"] - ref.stats["spikes_cooled_down"]
