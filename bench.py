"""Benchmark: fused two-tier decode attention, us/layer and achieved HBM GB/s.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config c3_7b_16k_b8]

A step is one decode step over L distinct layers (each with its own device
blob, > 1 GB in total so the 256 MB Infinity Cache cannot hold the working
set); each layer call is one launch of the fused kernel.  The L calls are
captured once in a HIP graph and replayed; the timed region is K replays
bracketed by HIP events on the capture stream, after 300 ms of untimed
replays (the GPU's clocks settle) and the W warm-up replays.  Inputs are synthetic
(seeded Gaussian K/V with outlier channels, 2% spike tokens) and resident in
HBM before timing starts.

Prints one JSON line (rank 0).  ``value`` is the achieved algorithmic HBM
bandwidth in GB/s: the bytes one layer-call must move (valid near rows fp16
K+V, far E4M3 K + INT4 V + fp16 scale/zero, decode rows, q in / out, spike
outputs, near_valid; no credit for gated-V skipping) divided by the
per-layer time.  ``us_per_layer`` and ``pct_peak`` are reported beside it,
with a ``roofline`` object (traffic from the committed rocprof counter
summary), the box's streaming-read ceiling measured in-run, and a
``cpu_baseline``: the whole batch of one layer on the host cores, the
faster of the C oracle's dequant+SDPA formulation and the reference's
formulation in torch ops (dequant -> cat -> repeat_interleave -> SDPA), each
timed over 100 calls or 20 s.

Every other benchmark configuration is timed the same way in the same run
(``other_configs``), and the default run also carries ``e2e_c5``,
``generate`` and ``crossover``: brief forms of the modes below.

Other modes (each prints its own JSON line): ``--e2e`` (the C5 decode +
promotion loop), ``--generate`` (a tiny LM decoding through the closure,
eager against one HIP graph per decode step), ``--crossover`` (the fused
kernel against exact fp16 attention, 1K-32K, B=1 and B=8).
"""

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "decode-attn µs/layer + achieved HBM GB/s (% peak), 7B shapes 16K ctx, 1 GPU"
PEAK_GBS = 8000.0


def algorithmic_bytes(B, Hq, Hkv, D, R, F, n_dec, v_group=0):
    """Bytes one layer-call must move: near (valid) fp16 K+V, far fp8 K +
    INT4 V + fp16 scale/zero (one pair per token, or per 32-dim group with
    v_group = 32), decode fp16 K+V, fp16 q in / out, flags and tokens,
    near_valid."""
    per_head = R * D * 4 + F * (D + D // 2 + 4 * (D // v_group if v_group else 1)) + n_dec * D * 4
    return B * Hkv * per_head + 2 * B * Hq * D * 2 + B * Hq * 8 + Hkv * 4


def algorithmic_bytes_turbo(B, Hq, Hkv, D, R, F, n_dec):
    """As algorithmic_bytes with the TurboQuant far tier: 2-bit key indices,
    1-bit QJL signs, fp16 norm + gamma, 2-bit values, one fp16 scale per 32
    dims."""
    per_head = R * D * 4 + F * (D // 4 + D // 8 + 4 + D // 4 + 2 * (D // 32)) + n_dec * D * 4
    return B * Hkv * per_head + 2 * B * Hq * D * 2 + B * Hq * 8 + Hkv * 4


def read_traffic(path):
    """Per-launch HBM traffic from a committed rocprofv3 --pmc summary:
    lines 'fetch_bytes_per_launch: N' / 'write_bytes_per_launch: N'."""
    if not path or not os.path.exists(path):
        return None
    vals = {}
    with open(path) as f:
        for line in f:
            if ":" in line:
                k, v = line.split(":", 1)
                try:
                    vals[k.strip()] = float(v.strip().split()[0])
                except (ValueError, IndexError):
                    pass
    if "fetch_bytes_per_launch" in vals and "write_bytes_per_launch" in vals:
        return vals["fetch_bytes_per_launch"] + vals["write_bytes_per_launch"]
    return None


def _timed(fn, warm_iters=10, warm_s=5.0, iters=100, time_s=20.0):
    """Warm up (``warm_iters`` calls or ``warm_s`` seconds, whichever ends
    first; at least one), then time calls until ``iters`` calls or
    ``time_s`` seconds (at least one).  -> (seconds per call, calls timed)."""
    t0 = time.perf_counter()
    n = 0
    while n < warm_iters and (n == 0 or time.perf_counter() - t0 < warm_s):
        fn()
        n += 1
    reps = 0
    t0 = time.perf_counter()
    while reps < iters and (reps == 0 or time.perf_counter() - t0 < time_s):
        fn()
        reps += 1
    return (time.perf_counter() - t0) / reps, reps


def host_cpu():
    """(model name, logical CPUs this process may run on)."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return model, n


def cpu_baseline(c, q, dk, dv, D, turbo=None):
    """The C oracle's formulation (dequant + concat + SDPA, fp64 softmax;
    OpenMP over (b, q head) for the fp8 tier, numpy for TurboQuant) on the
    whole batch of one layer.  -> (seconds per call, calls timed)."""
    import oracle
    from oracle import turbo as oturbo

    if turbo is not None:
        args = [q, c["near_k"], c["near_v"], c["near_valid"]] + list(turbo["far"]) + [turbo["C"], dk, dv]
        fn = oturbo.attend_formulation
    else:
        args = [q, c["near_k"], c["near_v"], c["near_valid"], c["far_k"], c["far_v"], c["far_v_scale"],
                c["far_v_zero"], dk, dv]
        fn = oracle.attend_formulation
    return _timed(lambda: fn(*args))


def torch_cpu_baseline(torch, c, q, dk, dv, D, threads, turbo=None):
    """The reference's formulation with torch ops on the host cores
    (mlx_foveated.py:239-312): dequant the far tier, concatenate the valid
    near rows, decode rows and far rows, repeat_interleave K and V to the
    query heads, SDPA (fp32: the host has no fast fp16 path), on the whole
    batch of one layer with ``threads`` torch threads.  -> (seconds per
    call, calls timed)."""
    import torch.nn.functional as Fn

    from foveated_kv_amd.tier_cache import dequant_int4_per_token, e4m3_to_fp16

    torch.set_num_threads(threads)
    t = {n: torch.from_numpy(np.ascontiguousarray(a)) for n, a in c.items()}
    qt = torch.from_numpy(q).float()[:, :, None, :]
    mv = int(t["near_valid"].max())
    nk, nv = t["near_k"][:, :, :mv], t["near_v"][:, :, :mv]
    dkt = torch.from_numpy(dk) if dk is not None else None
    dvt = torch.from_numpy(dv) if dv is not None else None
    G = q.shape[1] // nk.shape[1]
    if turbo is not None:
        from foveated_kv_amd import turbo as tq

        far = [torch.from_numpy(np.ascontiguousarray(a)) for a in turbo["far"]]
        tc = turbo["tc"]

        def dequant():
            return tq.turbo_dequant_keys(*far[:4], tc), tq.turbo_dequant_values(far[4], far[5])
    else:
        def dequant():
            return e4m3_to_fp16(t["far_k"]), dequant_int4_per_token(t["far_v"], t["far_v_scale"], t["far_v_zero"])

    def run():
        fk, fv = dequant()
        ks = [nk] + ([dkt] if dkt is not None else []) + [fk]
        vs = [nv] + ([dvt] if dvt is not None else []) + [fv]
        ak = torch.cat(ks, dim=2).float().repeat_interleave(G, dim=1)
        av = torch.cat(vs, dim=2).float().repeat_interleave(G, dim=1)
        return Fn.scaled_dot_product_attention(qt, ak, av, scale=D ** -0.5)

    with torch.no_grad():
        return _timed(run)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", default="c3_7b_16k_b8")
    ap.add_argument("--context", type=int, default=0,
                    help="run --config at this context length instead of its own (profiling: the same "
                         "kernel over another number of tiles)")
    ap.add_argument("--layers", type=int, default=0, help="distinct layer blobs (0: enough for > 1 GB)")
    ap.add_argument("--spikes", type=float, default=0.02)
    ap.add_argument("--e2e", action="store_true",
                    help="C5 end-to-end loop instead of the kernel line: importance partition + compress, then "
                         "--e2e-steps decode steps of attention + spike drain + promotion on one 64K layer")
    ap.add_argument("--e2e-steps", type=int, default=128)
    ap.add_argument("--spike-k", type=int, default=32,
                    help="--e2e: spiking far tokens per head per step (C5: up to 32; 1 = the reference's one)")
    ap.add_argument("--budget", type=int, default=0,
                    help="--e2e: promotions per drain (0: spike_k x H_kv, so the per-head limit binds)")
    ap.add_argument("--generate", action="store_true",
                    help="model decode loop instead of the kernel line: a seeded tiny LM (tests/_tiny_lm.py) "
                         "decoding through generate_fused, eager closure vs one HIP graph per decode step")
    ap.add_argument("--gen-tokens", type=int, default=128)
    ap.add_argument("--gen-layers", type=int, default=16)
    ap.add_argument("--gen-context", type=int, default=4096)
    ap.add_argument("--crossover", action="store_true",
                    help="kernel crossover instead of the kernel line: fused kernel vs exact fp16 torch SDPA on "
                         "the same GPU, 7B shapes, --cross-contexts x --cross-batches")
    ap.add_argument("--cross-contexts", type=int, nargs="+", default=[1024, 2048, 4096, 8192, 16384, 32768])
    ap.add_argument("--cross-batches", type=int, nargs="+", default=[1, 8])
    ap.add_argument("--no-group32", action="store_true",
                    help="C3 configs: skip the group-32 V layout measured beside the per-token headline")
    ap.add_argument("--v-group", type=int, default=0, choices=(0, 32),
                    help="fp8 far tier V: INT4 scale/zero per token (0) or per 32-dim group (32)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--stamps-spike-k", type=int, default=1,
                    help="--phase-stamps: spike_k of the handle; above 1 the top-K candidates kernel's phases "
                         "are reported too")
    ap.add_argument("--phase-stamps", action="store_true",
                    help="per-workgroup phase timeline of --config's kernel from the phase-stamp build "
                         "(make -C foveated_kv_amd/csrc STAMPS=1)")
    ap.add_argument("--no-e2e", action="store_true",
                    help="skip the C5 end-to-end step of the default run (e2e_c5)")
    ap.add_argument("--no-generate", action="store_true",
                    help="skip the whole-model decode of the default run (generate)")
    ap.add_argument("--no-crossover", action="store_true",
                    help="skip the kernel crossover of the default run (crossover)")
    ap.add_argument("--no-other-configs", action="store_true",
                    help="skip timing the other benchmark configurations (reported under other_configs)")
    ap.add_argument("--other-steps", type=int, default=30, help="timed steps per other configuration")
    ap.add_argument("--traffic", default=os.path.join(ROOT, "profiles", "attn_c3_16k_b8_traffic.txt"))
    ap.add_argument("--seed", type=int, default=1234)
    ap.add_argument("--eager", action="store_true",
                    help="time eager launches instead of a captured HIP graph (for counter collection)")
    ap.add_argument("--no-read-ceiling", action="store_true", help="skip the in-run HBM read-ceiling probe")
    ap.add_argument("--read-sweep", action="store_true",
                    help="with --copy-mib: sweep the read probe over launch shapes (else the best known one)")
    ap.add_argument("--copy-mib", type=int, default=0,
                    help="also time a plain device copy of this many MiB (HBM calibration; reported "
                         "as copy_gbs, read + write bytes)")
    args = ap.parse_args()
    if args.phase_stamps:  # the phase-stamp build of the library (make -C foveated_kv_amd/csrc STAMPS=1)
        os.environ["FKV_LIBRARY"] = os.path.join(ROOT, "foveated_kv_amd", "libfkv_stamps.so")

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(json.dumps({"error": "this build runs on one GPU: the decode path shards by (batch, kv_head) "
                                   "with no collective, so there is no multi-GPU figure; run with --gpus 1"}))
        sys.exit(2)

    import torch

    import oracle
    from foveated_kv_amd import _lib, ext, synthetic

    _lib.load()
    if not torch.cuda.is_available():
        raise SystemExit("bench.py needs a ROCm GPU")
    dev = torch.device("cuda:0")
    if args.e2e:
        run_e2e(args, torch, dev)
        return
    if args.generate:
        run_generate(args, torch, dev)
        return
    if args.crossover:
        run_crossover(args, torch, dev)
        return
    if args.phase_stamps:
        run_phase_stamps(args, torch, dev)
        return
    B, Hq, Hkv, D, S, n_dec = synthetic.CONFIGS[args.config]
    S = args.context or S
    cfg = ext.TierConfig()
    cfg.promo_headroom_min = 8
    turbo = args.config.startswith("c4_turbo")
    cfg.v_group = 0 if turbo else args.v_group
    tb = ext.tier_boundaries_c(cfg, S)
    R, F = tb["R_actual"], tb["far_count"]

    print(f"[bench] config {args.config}: B={B} Hq={Hq} Hkv={Hkv} D={D} S={S} n_dec={n_dec} "
          f"R={R} F={F}", file=sys.stderr, flush=True)
    k, v = synthetic.make_kv(B, Hkv, S, D, args.seed)
    q = synthetic.make_query(B, Hq, D, args.seed)
    synthetic.inject_spikes(k, q, tb["mid_start"], F, args.spikes, args.seed)
    dk, dv = synthetic.make_decode(B, Hkv, n_dec, D, args.seed)
    kt = torch.from_numpy(k).to(dev)
    vt = torch.from_numpy(v).to(dev)
    cl = ext.CompressHandle(cfg).compress_layer(kt, vt, with_archive=turbo)
    # the published C3 configuration names the group-32 V layout: measured beside the
    # reference's per-token layout in the same run (not the headline value)
    g32_side = args.config.startswith("c3_") and cfg.v_group == 0 and not args.no_group32
    if g32_side:
        cfg32 = ext.TierConfig()
        cfg32.promo_headroom_min = 8
        cfg32.v_group = 32
        cl32 = ext.CompressHandle(cfg32).compress_layer(kt, vt, with_archive=False)
    del kt, vt
    if turbo:
        from foveated_kv_amd import turbo as tq

        tc = tq.get_turbo_constants(D)
        tfar = tq.turbo_compress_keys(cl.archive_k, tc) + tq.turbo_compress_values(cl.archive_v)
        cl.archive_k = cl.archive_v = None

        def make_handle():
            return tq.TurboFoveatedHandle(cl.near_k, cl.near_v, *tfar, cl.near_valid, tc.Pi, tc.S, tc.centroids,
                                          spike_margin=10.0)
    else:
        def make_handle():
            return ext.FoveatedHandle(cl.near_k, cl.near_v, cl.far_k, cl.far_v, cl.far_v_scale, cl.far_v_zero,
                                      cl.near_valid, spike_margin=10.0)
    qt = torch.from_numpy(q).to(dev)[:, :, None, :]
    dkt = torch.from_numpy(dk).to(dev) if dk is not None else None
    dvt = torch.from_numpy(dv).to(dev) if dv is not None else None

    nbytes = (algorithmic_bytes_turbo(B, Hq, Hkv, D, R, F, n_dec) if turbo
              else algorithmic_bytes(B, Hq, Hkv, D, R, F, n_dec, cfg.v_group))
    L, blob_bytes, ms_step = time_layers(torch, dev, make_handle, args.layers, qt, dkt, dvt, args.steps,
                                         args.warmup, args.eager)
    us_layer = ms_step * 1000.0 / L
    gbs = nbytes / (us_layer * 1e-6) / 1e9
    print(f"[bench] {L} layer blobs x {blob_bytes / 2**20:.1f} MiB; algorithmic {nbytes / 1e6:.2f} MB/layer; "
          f"{us_layer:.3f} us/layer", file=sys.stderr, flush=True)

    result = {
        "metric": METRIC,
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16 operands, f32 accumulation",
        "data": "synthetic",
        "config": {"workload": args.config, "B": B, "Hq": Hq, "Hkv": Hkv, "D": D, "context": S,
                   "near_valid": R, "far": F, "n_decode": n_dec, "layers_per_step": L,
                   "spike_frac": args.spikes,
                   "far_format": ("turboquant 2-bit K + 1-bit QJL, 2-bit V group-32" if turbo
                                  else "fp8-e4m3 K + int4 group-32 V" if cfg.v_group
                                  else "fp8-e4m3 K + int4 per-token V")},
        "us_per_layer": round(us_layer, 3),
        "launch": "eager" if args.eager else "hip-graph",
        "clock_settle_ms": SETTLE_MS,
        "pct_peak": round(100.0 * gbs / PEAK_GBS, 2),
    }
    if g32_side:
        def make32():
            return ext.FoveatedHandle(cl.near_k, cl.near_v, cl32.far_k, cl32.far_v, cl32.far_v_scale,
                                      cl32.far_v_zero, cl.near_valid, spike_margin=10.0)
        L32, _, ms32 = time_layers(torch, dev, make32, args.layers, qt, dkt, dvt, args.steps, args.warmup,
                                   args.eager)
        b32 = algorithmic_bytes(B, Hq, Hkv, D, R, F, n_dec, 32)
        us32 = ms32 * 1000.0 / L32
        result["group32_v"] = {"far_format": "fp8-e4m3 K + int4 group-32 V", "us_per_layer": round(us32, 3),
                               "gbs": round(b32 / (us32 * 1e-6) / 1e9, 2),
                               "pct_peak": round(100.0 * b32 / (us32 * 1e-6) / 1e9 / PEAK_GBS, 2),
                               "algorithmic_bytes": b32, "layers_per_step": L32}
        del cl32
    traffic = read_traffic(args.traffic) if args.config == "c3_7b_16k_b8" and not cfg.v_group else None
    result["roofline"] = {"bound": "hbm", "achieved": round(gbs, 2), "peak": PEAK_GBS, "unit": "GB/s",
                          "frac": round(gbs / PEAK_GBS, 4), "traffic": traffic,
                          "algorithmic_bytes": nbytes}
    if not args.no_cpu_baseline:
        c = {n: getattr(cl, n).cpu().numpy() for n in ("near_k", "near_v", "far_k", "far_v", "far_v_scale",
                                                        "far_v_zero", "near_valid")}
        tb_ = None
        if turbo:
            from oracle import turbo as oturbo

            tb_ = {"far": [t.cpu().numpy() for t in tfar], "C": oturbo.constants(D), "tc": tc}
        threads = int(os.environ.get("OMP_NUM_THREADS", "0")) or host_cpu()[1]
        cpu_model, nproc = host_cpu()
        dt_o, reps_o = cpu_baseline(c, q, dk, dv, D, turbo=tb_)
        dt_t, reps_t = torch_cpu_baseline(torch, c, q, dk, dv, D, threads, turbo=tb_)
        best = min(dt_o, dt_t)
        result["cpu_baseline"] = {
            "value": round(nbytes / best / 1e9, 4), "unit": "GB/s", "cores": threads, "kind": "port",
            "us_per_layer": round(best * 1e6, 1),
            "sample": f"the whole batch (B={B}) of one layer of {args.config}, the faster of two host "
                      f"formulations; each warmed for 10 calls or 5 s, then timed over 100 calls or 20 s, "
                      f"whichever ends first",
            "cpu_model": cpu_model, "nproc": nproc,
            "formulations": {
                "oracle_c": {"us_per_layer": round(dt_o * 1e6, 1), "calls": reps_o,
                             "what": "C oracle dequant + concat + SDPA, fp64 softmax, " +
                                     ("numpy" if turbo else f"OpenMP over (b, q head), {threads} threads")},
                "torch_cpu": {"us_per_layer": round(dt_t * 1e6, 1), "calls": reps_t,
                              "what": f"torch dequant -> cat -> repeat_interleave -> SDPA (fp32), "
                                      f"{threads} threads"}},
        }
    if not args.no_other_configs:
        # every other benchmark configuration, timed the same way in this run
        # (fewer steps; not the headline value)
        others = {}
        for name in synthetic.CONFIGS:
            if name == args.config:
                continue
            others[name] = config_line(torch, dev, ext, synthetic, name, args.other_steps, 5, args.seed,
                                       args.spikes, args.eager)
            print(f"[bench] {name}: {others[name]['us_per_layer']} us/layer, {others[name]['gbs']} GB/s",
                  file=sys.stderr, flush=True)
        # C1 as BASELINE names it: importance partition, per-head-scaled fp8
        # K, INT4 V in groups of 32 (the line above keeps the reference's
        # formats, recency partition, unscaled K, per-token V)
        name = "c1_qwen05b_512"
        if name != args.config:
            key = name + "_scaled_k_g32"
            others[key] = config_line(torch, dev, ext, synthetic, name, args.other_steps, 5, args.seed,
                                      args.spikes, args.eager, v_group=32, k_scale=True, importance=True)
            print(f"[bench] {key}: {others[key]['us_per_layer']} us/layer, {others[key]['gbs']} GB/s",
                  file=sys.stderr, flush=True)
        result["other_configs"] = others
    if not args.no_e2e and not args.no_other_configs:
        # the C5 decode step end to end (attention, spike drain, promotion),
        # graph-replayed, with C5's up to 32 tokens per head and with the
        # reference's single token (bench.py --e2e: the full comparison)
        # (a failure here is reported in the field; the headline line stands)
        try:
            result["e2e_c5"] = run_e2e(args, torch, dev, brief=True)
            print(f"[bench] e2e_c5: {result['e2e_c5']['us_per_step']} us/step (spike_k {args.spike_k}), "
                  f"{result['e2e_c5']['reference_single_token']['us_per_step']} us/step (spike_k 1)",
                  file=sys.stderr, flush=True)
        except Exception as e:  # noqa: BLE001
            result["e2e_c5"] = {"error": f"{type(e).__name__}: {e}"}
            print(f"[bench] e2e_c5 failed: {e!r}", file=sys.stderr, flush=True)
    # the whole-model decode (a tiny LM through the patched closure, one HIP
    # graph per token) and the kernel crossover against exact fp16 attention,
    # in the default run too (bench.py --generate / --crossover print them alone)
    for key, flag, fn in (("generate", args.no_generate, run_generate),
                          ("crossover", args.no_crossover, run_crossover)):
        if flag or args.no_other_configs:
            continue
        try:
            result[key] = fn(args, torch, dev, brief=True)
            print(f"[bench] {key} done", file=sys.stderr, flush=True)
        except Exception as e:  # noqa: BLE001
            result[key] = {"error": f"{type(e).__name__}: {e}"}
            print(f"[bench] {key} failed: {e!r}", file=sys.stderr, flush=True)
    if args.copy_mib:
        result["copy_gbs"] = copy_bandwidth(torch, dev, args.copy_mib)
        result["read_ceiling_gbs"], result["read_ceiling_launch"] = read_ceiling(torch, dev, args.copy_mib,
                                                                                 sweep=args.read_sweep)
    elif not args.no_read_ceiling:
        # this box's streaming-read ceiling, measured beside the kernel
        result["read_ceiling_gbs"], _ = read_ceiling(torch, dev, 2048, sweep=False)
    print(json.dumps(result), flush=True)


SETTLE_MS = 300.0


def config_line(torch, dev, ext, synthetic, name, steps, warmup, seed, spikes, eager, v_group=0, k_scale=False,
                importance=False):
    """One benchmark configuration timed like the headline (distinct layer
    blobs, HIP-graph replays, HIP events): us per layer and algorithmic
    GB/s of the reference's per-token V layout (TurboQuant for C4), or of
    group-32 V / per-head-scaled K / the importance partition when asked."""
    B, Hq, Hkv, D, S, n_dec = synthetic.CONFIGS[name]
    cfg = ext.TierConfig()
    cfg.promo_headroom_min = 8
    cfg.v_group = v_group
    cfg.k_scale = 1 if k_scale else 0
    turbo = name.startswith("c4_turbo")
    tb = ext.tier_boundaries_c(cfg, S)
    R, F = tb["R_actual"], tb["far_count"]
    k, v = synthetic.make_kv(B, Hkv, S, D, seed)
    q = synthetic.make_query(B, Hq, D, seed)
    imp = None
    if importance:
        imp = torch.from_numpy(synthetic.make_importance(B, Hkv, S, seed)).to(dev)
        _, fidx = ext.partition_importance(cfg, imp, B, Hkv, S)
        synthetic.inject_spikes_at(k, q, fidx.cpu().numpy(), spikes, seed)
    else:
        synthetic.inject_spikes(k, q, tb["mid_start"], F, spikes, seed)
    dk, dv = synthetic.make_decode(B, Hkv, n_dec, D, seed)
    cl = ext.CompressHandle(cfg).compress_layer(torch.from_numpy(k).to(dev), torch.from_numpy(v).to(dev),
                                                with_archive=turbo, importance=imp)
    if turbo:
        from foveated_kv_amd import turbo as tq

        tc = tq.get_turbo_constants(D)
        tfar = tq.turbo_compress_keys(cl.archive_k, tc) + tq.turbo_compress_values(cl.archive_v)
        cl.archive_k = cl.archive_v = None

        def make_handle():
            return tq.TurboFoveatedHandle(cl.near_k, cl.near_v, *tfar, cl.near_valid, tc.Pi, tc.S, tc.centroids,
                                          spike_margin=10.0)
    else:
        def make_handle():
            return ext.FoveatedHandle(cl.near_k, cl.near_v, cl.far_k, cl.far_v, cl.far_v_scale, cl.far_v_zero,
                                      cl.near_valid, spike_margin=10.0, far_k_scale=cl.far_k_scale)
    qt = torch.from_numpy(q).to(dev)[:, :, None, :]
    dkt = torch.from_numpy(dk).to(dev) if dk is not None else None
    dvt = torch.from_numpy(dv).to(dev) if dv is not None else None
    nbytes = (algorithmic_bytes_turbo(B, Hq, Hkv, D, R, F, n_dec) if turbo
              else algorithmic_bytes(B, Hq, Hkv, D, R, F, n_dec, v_group) + (B * Hkv * 4 if k_scale else 0))
    L, _, ms = time_layers(torch, dev, make_handle, 0, qt, dkt, dvt, steps, warmup, eager)
    us = ms * 1000.0 / L
    gbs = nbytes / (us * 1e-6) / 1e9
    fmt = ("turboquant" if turbo else ("per-head-scaled " if k_scale else "") + "fp8-e4m3 K + int4 " +
           ("group-32" if v_group else "per-token") + " V" + (", importance partition" if importance else ""))
    return {"B": B, "Hq": Hq, "Hkv": Hkv, "D": D, "context": S, "n_decode": n_dec,
            "far_format": fmt,
            "us_per_layer": round(us, 3), "gbs": round(gbs, 2), "pct_peak": round(100.0 * gbs / PEAK_GBS, 2),
            "algorithmic_bytes": nbytes, "layers_per_step": L, "steps": steps}


def settle_clocks(torch, stream, step, min_ms=SETTLE_MS):
    """Untimed steps for ``min_ms`` of wall time before the warm-up steps.
    From an idle start MI355X runs this workload at a transient rate for the
    first tens of milliseconds of continuous work (measured from a cold
    process: ~46 us/layer for 5 steps, 54-59 us at steps 10-25, steady ~44.5
    us only after ~80 steps); a decode loop keeps the GPU busy, so the
    steady state is the one measured.  The timed region is unchanged."""
    t0 = time.perf_counter()
    while (time.perf_counter() - t0) * 1e3 < min_ms:
        with torch.cuda.stream(stream):
            for _ in range(20):
                step()
        torch.cuda.synchronize()


def time_layers(torch, dev, make_handle, layers, qt, dkt, dvt, steps, warmup, eager):
    """Build distinct layer handles (> 1 GiB of blobs unless ``layers``), run
    one decode step over all of them as a HIP graph (or eagerly), time
    ``steps`` steps with HIP events on the replay stream.  Returns (layers,
    blob bytes, ms per step); checks that a replay equals an eager call."""
    handles = []
    blob_bytes = None
    while True:
        h = make_handle()
        handles.append(h)
        blob_bytes = h.get_blob_info().blob_bytes
        if (layers and len(handles) >= layers) or (not layers and len(handles) * blob_bytes > (1 << 30)
                                                   and len(handles) >= 4):
            break
    # eager warm-up (allocates the split workspace outside graph capture)
    for h in handles:
        h(qt, dkt, dvt)
    torch.cuda.synchronize()
    stream = torch.cuda.Stream(device=dev)
    outs = []
    if eager:
        def step():
            for h in handles:
                h(qt, dkt, dvt)
        with torch.cuda.stream(stream):
            outs = [h(qt, dkt, dvt) for h in handles]
    else:
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.stream(stream):
            with torch.cuda.graph(graph, stream=stream):
                for h in handles:
                    outs.append(h(qt, dkt, dvt))
        step = graph.replay
    torch.cuda.synchronize()
    settle_clocks(torch, stream, step)
    with torch.cuda.stream(stream):
        for _ in range(warmup):
            step()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        start.record(stream)
        for _ in range(steps):
            step()
        end.record(stream)
    torch.cuda.synchronize()
    ms_step = start.elapsed_time(end) / steps
    # sanity: graph output equals eager output for layer 0
    ref = handles[0](qt, dkt, dvt)
    torch.cuda.synchronize()
    assert torch.equal(ref[0], outs[0][0]) and torch.equal(ref[2], outs[0][2]), "graph replay diverged"
    return len(handles), blob_bytes, ms_step


def run_e2e(args, torch, dev, brief=False):
    """Workload C5: compress + decode + promote on one 70B-like layer (Hq=64,
    Hkv=8, D=128, 64K context, B=1).  Seeded importance partition, 2 % of
    far tokens aligned with the group query, per-step query drift, one
    decode token appended per step, spike drain (GQA dedup, cooldown 5, up
    to --spike-k far tokens per KV head and step -- C5's "up to 32 far
    tokens per head per step" -- within a budget of --budget per drain) and
    promotion of exact fp16 rows from the pinned host archive -- on the
    device, and again with a host-side drain for comparison.  Prints one JSON
    line: us per decode step of the graph-replayed device-drain loop, with
    the same loop reading the archive from HBM instead of pinned host memory,
    the eager device-drain loop, the host-drain loop and the reference's
    single-token drain (spike_k 1, budget 8) beside it, and the promotions
    per step of each.  brief: the two graph-replayed loops only (--spike-k
    tokens, and the reference's single token), returned as a dict for the
    default run's line instead of printed."""
    from foveated_kv_amd import ext, synthetic
    from foveated_kv_amd.promotion import PromotionPipeline

    B, Hq, Hkv, D, S, _ = synthetic.CONFIGS["c5_70b_64k"]
    steps, seed = args.e2e_steps, args.seed
    cfg = ext.TierConfig()
    cfg.promo_headroom_min = 8
    cfg.v_group = args.v_group
    k, v = synthetic.make_kv(B, Hkv, S, D, seed)
    q0 = synthetic.make_query(B, Hq, D, seed)
    imp = torch.from_numpy(synthetic.make_importance(B, Hkv, S, seed)).to(dev)
    _, far_idx = ext.partition_importance(cfg, imp, B, Hkv, S)
    far_idx = far_idx.cpu().numpy()
    synthetic.inject_spikes_at(k, q0, far_idx, args.spikes, seed)
    qs = torch.from_numpy(synthetic.drift_queries(q0, steps, 0.05, seed)).to(dev)[:, :, :, None, :]
    dk, dv = synthetic.make_decode(B, Hkv, steps, D, seed)
    dkt, dvt = torch.from_numpy(dk).to(dev), torch.from_numpy(dv).to(dev)
    kt, vt = torch.from_numpy(k).to(dev), torch.from_numpy(v).to(dev)
    spike_k = args.spike_k
    budget = args.budget if args.budget > 0 else spike_k * Hkv
    print(f"[e2e] C5 B={B} Hq={Hq} Hkv={Hkv} D={D} S={S} steps={steps} spike_k={spike_k} budget={budget}",
          file=sys.stderr, flush=True)

    def compress(kk=1):
        cl = ext.CompressHandle(cfg).compress_layer(kt, vt, importance=imp)
        h = ext.FoveatedHandle(cl.near_k, cl.near_v, cl.far_k, cl.far_v, cl.far_v_scale, cl.far_v_zero,
                               cl.near_valid, spike_margin=10.0, spike_k=kk)
        return cl, h

    compress()  # warm (module load, first launches)
    torch.cuda.synchronize()
    fdev = torch.from_numpy(far_idx).to(dev).contiguous()

    def loop(device_drain, kk, bud):
        """One compress + `steps` decode steps; returns timings and the
        promotion outcome.  device_drain: the filter and the row copies run as
        a kernel after each attention launch (no host round trip); else the
        spike outputs are read back and drained on the host, as the
        reference does."""
        t0 = time.perf_counter()
        cl, h = compress(kk)
        torch.cuda.synchronize()
        compress_ms = (time.perf_counter() - t0) * 1e3
        pipe = PromotionPipeline(1, cooldown_steps=5, max_per_drain=bud, spike_k=kk)
        pipe.register_archive_tensors(0, cl.archive_k, cl.archive_v, far_idx)
        pipe.register_blob(0, h)
        h(qs[0], dkt[:, :, :1], dvt[:, :, :1])  # allocates the call's split workspace
        torch.cuda.synchronize()
        t_call = t_drain = 0.0
        t0 = time.perf_counter()
        for t in range(steps):
            ta = time.perf_counter()
            if not device_drain:
                pipe.order(0)
            # the decode buffer as a step sees it: views of one preallocated buffer
            out, flags, toks = h(qs[t], dkt[:, :, :t + 1], dvt[:, :, :t + 1])
            tb_ = time.perf_counter()
            if device_drain:
                pipe.drain_spikes_device(0, flags, toks, fdev, t)
            else:
                both = torch.cat([flags.reshape(-1), toks.reshape(-1)]).cpu().numpy()  # one copy, then the filter
                pipe.drain_spikes(0, both[:flags.numel()].reshape(tuple(flags.shape)), both[flags.numel():],
                                  far_idx, t)
            t_call += tb_ - ta
            t_drain += time.perf_counter() - tb_
        pipe.synchronize()
        torch.cuda.synchronize()
        loop_s = time.perf_counter() - t0
        return {"us_per_step": loop_s / steps * 1e6, "compress_ms": compress_ms, "cl": cl, "h": h,
                "host_call_us": t_call / steps * 1e6, "host_drain_us": t_drain / steps * 1e6,
                "stats": pipe.get_stats(), "near_valid_end": h.read_near_valid()}

    def loop_graph(kk, bud, hbm_archive=False):
        """The device-drain loop with the decode step captured once in a HIP
        graph: with n (a device int32) the step's decode-row count, gather the
        query of step n - 1, attention over the fixed-capacity decode buffer,
        the drain kernel with n as its step (the filter only compares steps,
        so the +1 offset changes nothing), which then advances n.  Step 0
        runs eagerly (it sizes the workspaces), steps 1.. are graph replays
        with nothing read back.  hbm_archive: the archive rows stay in device
        memory (register_archive_tensors(device=True)) instead of pinned host
        memory."""
        t0 = time.perf_counter()
        cl, h = compress(kk)
        torch.cuda.synchronize()
        compress_ms = (time.perf_counter() - t0) * 1e3
        pipe = PromotionPipeline(1, cooldown_steps=5, max_per_drain=bud, spike_k=kk)
        pipe.register_archive_tensors(0, cl.archive_k, cl.archive_v, far_idx, device=hbm_archive)
        pipe.register_blob(0, h)
        n_d = torch.ones(1, dtype=torch.int32, device=dev)
        q1 = torch.cat([qs[:1], qs])  # row n holds the query of step n - 1
        q_d = torch.empty((1,) + tuple(qs.shape[1:]), dtype=qs.dtype, device=dev)

        def one():
            torch.index_select(q1, 0, n_d, out=q_d)
            out, flags, toks = h(q_d[0], dkt, dvt, n_decode=n_d)
            pipe.drain_spikes_device(0, flags, toks, fdev, n_d, advance_step=True)
            return out

        one()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            one()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(1, steps):
            g.replay()
        torch.cuda.synchronize()
        loop_s = time.perf_counter() - t0
        assert int(n_d.item()) == steps + 1, "graph replays did not advance the step counter"
        return {"us_per_step": loop_s / max(steps - 1, 1) * 1e6, "compress_ms": compress_ms,
                "stats": pipe.get_stats(), "near_valid_end": h.read_near_valid()}

    if brief:
        gres = loop_graph(spike_k, budget)
        g1res = loop_graph(1, 8) if spike_k != 1 or budget != 8 else gres
        return {"workload": "c5_70b_64k_e2e", "steps": steps - 1,
                "launch": "one HIP graph replay per step (query gather, attention, drain + step advance)",
                "spike_k": spike_k, "budget_per_drain": budget,
                "us_per_step": round(gres["us_per_step"], 2),
                "promotions_per_step": round(gres["stats"]["promotions_completed"] / steps, 3),
                "near_valid_end": gres["near_valid_end"],
                "reference_single_token": {"spike_k": 1, "budget_per_drain": 8,
                                           "us_per_step": round(g1res["us_per_step"], 2),
                                           "promotions_per_step":
                                               round(g1res["stats"]["promotions_completed"] / steps, 3)}}
    dres = loop(True, spike_k, budget)
    hres = loop(False, spike_k, budget)
    gres = loop_graph(spike_k, budget)
    hbres = loop_graph(spike_k, budget, hbm_archive=True)
    g1res = loop_graph(1, 8) if spike_k != 1 or budget != 8 else gres
    cl, h = dres["cl"], dres["h"]
    # device time of the attention call on the final state (queued back to back)
    dk_end, dv_end = dkt.contiguous(), dvt.contiguous()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(20):
        h(qs[-1], dk_end, dv_end)
    e1.record()
    torch.cuda.synchronize()
    attn_us = e0.elapsed_time(e1) * 1e3 / 20
    result = {
        "metric": "C5 end-to-end decode step (attention + spike drain + promotion), 70B-like layer, 64K ctx, 1 GPU",
        "value": round(gres["us_per_step"], 2), "unit": "us/step", "n_gpus": 1, "steps": steps - 1, "warmup": 1,
        "ms_per_step": round(gres["us_per_step"] / 1e3, 5), "higher_is_better": False, "scaling": "weak",
        "vs_baseline": None, "dtype": "f16 operands, f32 accumulation", "data": "synthetic",
        "config": {"workload": "c5_70b_64k_e2e", "B": B, "Hq": Hq, "Hkv": Hkv, "D": D, "context": S,
                   "near_valid": int(cl.near_valid[0]), "far": int(cl.far_k.shape[2]),
                   "headroom": int(cl.near_k.shape[2] - cl.near_valid[0]), "spike_frac": args.spikes,
                   "partition": "importance (seeded N(0,1) scores)", "query_drift_eps": 0.05,
                   "drain": "device (filter + row copies in one kernel after each attention launch)",
                   "launch": "one HIP graph replay per step (query gather, attention, drain + step advance); "
                             "step 0 eager",
                   "far_format": "fp8-e4m3 K + int4 group-32 V" if args.v_group else "fp8-e4m3 K + int4 per-token V"},
        "compress_ms": round(gres["compress_ms"], 3),
        "attn_us_device": round(attn_us, 3),
        "spike_k": spike_k, "budget_per_drain": budget,
        "promotions_per_step": round(gres["stats"]["promotions_completed"] / steps, 3),
        "promotion_stats": gres["stats"],
        "near_valid_end": gres["near_valid_end"],
        "eager_device_drain": {"us_per_step": round(dres["us_per_step"], 2),
                               "host_us_per_step": {"attention_call": round(dres["host_call_us"], 2),
                                                    "drain_launch": round(dres["host_drain_us"], 2)},
                               "same_promotions": gres["stats"] == dres["stats"]
                               and gres["near_valid_end"] == dres["near_valid_end"]},
        "archive_in_hbm": {"us_per_step": round(hbres["us_per_step"], 2),
                           "same_promotions": hbres["stats"] == gres["stats"]
                           and hbres["near_valid_end"] == gres["near_valid_end"]},
        "reference_single_token": {"spike_k": 1, "budget_per_drain": 8,
                                   "us_per_step": round(g1res["us_per_step"], 2),
                                   "promotions_per_step": round(g1res["stats"]["promotions_completed"] / steps, 3),
                                   "promotion_stats": g1res["stats"]},
        "host_drain": {"us_per_step": round(hres["us_per_step"], 2),
                       "host_us_per_step": {"attention_call": round(hres["host_call_us"], 2),
                                            "spike_readback_drain_and_flush": round(hres["host_drain_us"], 2)},
                       "same_promotions": hres["stats"] == gres["stats"]
                       and hres["near_valid_end"] == gres["near_valid_end"]},
    }
    print(json.dumps(result), flush=True)


def run_phase_stamps(args, torch, dev):
    """Where one launch's time goes, from the phase-stamp build: --config's
    handle (TurboQuant for C4) is called back to back for 300 ms, then
    --steps more times; the stamps of the last launch (100 MHz clock, per
    workgroup: entry, prologue done, each wave's stream done, records
    published, arrival counted, the last split's merge done; the XCD id)
    become one JSON line of phase durations in us: p50 / max over
    workgroups, the spread of the XCDs' first starts and last stream ends,
    and the last output relative to the first workgroup's entry."""
    import ctypes

    from foveated_kv_amd import _lib, ext

    lib = _lib.load()
    probe = (ctypes.c_uint64 * 64)()
    if lib.fkv_phase_stamps(ctypes.cast(probe, ctypes.c_void_p), 0, 1) != 0:
        raise SystemExit("the library has no phase stamps: build it with make -C foveated_kv_amd/csrc STAMPS=1")
    name = args.config
    B, Hq, Hkv, D, S, n_dec = __import__("foveated_kv_amd.synthetic", fromlist=["CONFIGS"]).CONFIGS[name]
    make_handle, qt, dkt, dvt, _ = config_handles(torch, dev, ext, name, args.seed, args.spikes)
    h = make_handle()
    if args.stamps_spike_k > 1:
        h.set_spike_k(args.stamps_spike_k)
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < SETTLE_MS / 1e3:
        for _ in range(20):
            h(qt, dkt, dvt)
        torch.cuda.synchronize()
    for _ in range(max(args.steps, 1)):
        h(qt, dkt, dvt)
    torch.cuda.synchronize()
    n_wgs = 8192
    raw = (ctypes.c_uint64 * (64 * n_wgs))()
    _lib.check(lib.fkv_phase_stamps(ctypes.cast(raw, ctypes.c_void_p), n_wgs, 1), "fkv_phase_stamps")
    st = np.frombuffer(raw, dtype=np.uint64).reshape(n_wgs, 64).astype(np.int64)
    st = st[st[:, 0] > 0]
    t_first = st[:, 0].min()
    us = lambda x: np.asarray(x, np.float64) / 100.0  # 100 MHz ticks -> us
    waves = [c for c in range(2, 18) if (st[:, c] > 0).any()]
    wave_end = st[:, waves].max(axis=1)
    xcc = st[:, 63]
    # slot 22 is written only by the last split of a row to arrive, which
    # varies between launches: keep the stamps of this launch (after its arrival)
    merged = st[st[:, 22] > st[:, 21]]

    def pq(x):
        x = np.asarray(x, np.float64)
        return {"p50": round(float(np.median(x)), 3), "max": round(float(x.max()), 3)} if x.size else None

    ends = {int(x): us(wave_end[xcc == x].max() - t_first) for x in np.unique(xcc)}
    starts = {int(x): us(st[xcc == x, 0].min() - t_first) for x in np.unique(xcc)}
    out = {
        "mode": "phase-stamps", "config": name, "workgroups": int(len(st)), "waves_per_wg": len(waves),
        "launches_before": args.steps, "unit": "us",
        "entry_spread": pq(us(st[:, 0] - t_first)),
        "xcd_first_start": {k: round(v, 3) for k, v in sorted(starts.items())},
        "prologue": pq(us(st[:, 1] - st[:, 0])),
        "stream_to_last_wave": pq(us(wave_end - st[:, 1])),
        "xcd_last_stream_end": {k: round(v, 3) for k, v in sorted(ends.items())},
        "xcd_end_spread": round(max(ends.values()) - min(ends.values()), 3),
        "records_published": pq(us(st[:, 20] - wave_end)) if (st[:, 20] > 0).all() else None,
        "arrival": pq(us(st[:, 21] - st[:, 20])) if (st[:, 21] > 0).all() else None,
        "last_split_merge": pq(us(merged[:, 22] - merged[:, 21])) if len(merged) else None,
        "last_output": round(float(us(merged[:, 22].max() - t_first)), 3) if len(merged) else None,
        "last_stream_end": round(float(us(wave_end.max() - t_first)), 3),
    }
    if args.stamps_spike_k > 1:
        # the top-K candidates kernel's workgroups (slots 32..): entry, maxima
        # staged, cuts known, each wave's candidates done, the selection
        # slots 32 entry, 33 staged, 34 cuts, 35+w wave done, 39+w query
        # operands, 43+w last batch begun, 47 the quad's selection done (its
        # last workgroup; an older launch's stamp is earlier than this one's)
        sel = np.frombuffer(raw, dtype=np.uint64).reshape(n_wgs, 64).astype(np.int64)[:, 32:60]
        sel = sel[(sel[:, 0] > 0) & (sel[:, 3] > 0)]
        if len(sel):
            t0s = sel[:, 0].min()
            done = sel[:, 3:7].max(axis=1)
            selected = sel[:, 15] > done
            end = max(done.max(), sel[selected, 15].max()) if selected.any() else done.max()
            out["topk_candidates"] = {
                "workgroups": int(len(sel)), "spike_k": args.stamps_spike_k,
                "entry_spread": pq(us(sel[:, 0] - t0s)),
                "stage_maxima": pq(us(sel[:, 1] - sel[:, 0])),
                "cut_search": pq(us(sel[:, 2] - sel[:, 1])),
                "query_operands": pq(us((sel[:, 7:11] - sel[:, 2:3]).ravel())),
                "deal_and_full_batches": pq(us((sel[:, 11:15] - sel[:, 7:11]).ravel())),
                "last_batch": pq(us((sel[:, 3:7] - sel[:, 11:15]).ravel())),
                "rescore_and_append": pq(us(done - sel[:, 2])),
                "arrival_and_selection": pq(us(sel[selected, 15] - done[selected])) if selected.any() else None,
                # each wave's first batch (slots 48+w begun, 52+w rescored, 56+w slots reserved), where
                # it ran in this launch (its stamps after the wave's query operands)
                **first_batch_phases(sel, us, pq),
                "last_done": round(float(us(end - t0s)), 3),
                "start_after_attention_output": (round(float(us(t0s - merged[:, 22].max())), 3)
                                                 if len(merged) else None),
            }
    print(json.dumps(out), flush=True)


def first_batch_phases(sel, us, pq):
    """The top-K candidates kernel's first rescoring batch per wave, from
    its phase stamps (columns relative to slot 32): 16+w begun, 20+w
    rescored (loads and matrix instructions), 24+w slots reserved (one
    atomic per head); a wave's stamps count only where they follow its
    query-operand stamp (7+w) of this launch."""
    begun, resc, resv, qop = sel[:, 16:20], sel[:, 20:24], sel[:, 24:28], sel[:, 7:11]
    ok = (begun > qop) & (resc > begun) & (resv > resc)
    if not ok.any():
        return {}
    return {"first_batch_waves": int(ok.sum()),
            "first_batch_rescore": pq(us((resc - begun)[ok])),
            "first_batch_slot_reservation": pq(us((resv - resc)[ok])),
            "first_batch_begun_after_query": pq(us((begun - qop)[ok]))}


def config_handles(torch, dev, ext, name, seed, spikes):
    """make_handle, the query / decode tensors and the algorithmic bytes of
    one benchmark configuration (the inputs config_line times)."""
    from foveated_kv_amd import synthetic

    B, Hq, Hkv, D, S, n_dec = synthetic.CONFIGS[name]
    cfg = ext.TierConfig()
    cfg.promo_headroom_min = 8
    turbo = name.startswith("c4_turbo")
    tb = ext.tier_boundaries_c(cfg, S)
    R, F = tb["R_actual"], tb["far_count"]
    k, v = synthetic.make_kv(B, Hkv, S, D, seed)
    q = synthetic.make_query(B, Hq, D, seed)
    synthetic.inject_spikes(k, q, tb["mid_start"], F, spikes, seed)
    dk, dv = synthetic.make_decode(B, Hkv, n_dec, D, seed)
    cl = ext.CompressHandle(cfg).compress_layer(torch.from_numpy(k).to(dev), torch.from_numpy(v).to(dev),
                                                with_archive=turbo)
    if turbo:
        from foveated_kv_amd import turbo as tq

        tc = tq.get_turbo_constants(D)
        tfar = tq.turbo_compress_keys(cl.archive_k, tc) + tq.turbo_compress_values(cl.archive_v)

        def make_handle():
            return tq.TurboFoveatedHandle(cl.near_k, cl.near_v, *tfar, cl.near_valid, tc.Pi, tc.S, tc.centroids,
                                          spike_margin=10.0)
    else:
        def make_handle():
            return ext.FoveatedHandle(cl.near_k, cl.near_v, cl.far_k, cl.far_v, cl.far_v_scale, cl.far_v_zero,
                                      cl.near_valid, spike_margin=10.0)
    qt = torch.from_numpy(q).to(dev)[:, :, None, :]
    dkt = torch.from_numpy(dk).to(dev) if dk is not None else None
    dvt = torch.from_numpy(dv).to(dev) if dv is not None else None
    nbytes = (algorithmic_bytes_turbo(B, Hq, Hkv, D, R, F, n_dec) if turbo
              else algorithmic_bytes(B, Hq, Hkv, D, R, F, n_dec))
    return make_handle, qt, dkt, dvt, nbytes


def time_graph(torch, dev, fns, steps, warmup):
    """Capture one call of every function in ``fns`` in a HIP graph, settle
    the clocks, replay ``warmup`` times, then time ``steps`` replays with HIP
    events on the replay stream.  -> ms per replay."""
    for fn in fns:  # eager first call (workspaces, library handles) outside capture
        fn()
    torch.cuda.synchronize()
    stream = torch.cuda.Stream(device=dev)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            for fn in fns:
                fn()
    torch.cuda.synchronize()
    settle_clocks(torch, stream, graph.replay)
    with torch.cuda.stream(stream):
        for _ in range(warmup):
            graph.replay()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        start.record(stream)
        for _ in range(steps):
            graph.replay()
        end.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


def run_crossover(args, torch, dev, brief=False):
    """Kernel crossover (benchmark_crossover.py:45-82 of the reference, on
    one GPU): one decode attention call at 7B shapes (Hq=32, Hkv=8, D=128),
    exact fp16 attention over all S tokens against the fused kernel over the
    compressed tiers of the same tokens (10 % near fp16, 90 % far fp8 K +
    INT4 V).  Each side runs over distinct per-layer copies (>= 1 GiB in
    total, at most 256 layers) captured in one HIP graph, so neither reads a
    warm cache; the time is per layer.  Exact attention is timed three ways
    and the fastest counts: torch SDPA with native GQA (``enable_gqa``), the
    reference's formulation (``repeat_interleave`` + SDPA), and an explicit
    fp16 GEMM formulation (K q^T, fp32 softmax, P V; no copies of K or V).
    SDPA is limited to its fused (flash / memory-efficient) backends."""
    import torch.nn.functional as Fn
    from torch.nn.attention import SDPBackend, sdpa_kernel

    from foveated_kv_amd import ext

    # SDPA's fused backends only: its math fallback runs batched products on
    # transposed views, which the explicit GEMM formulation below avoids
    fused_backends = [SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]
    Hq, Hkv, D = 32, 8, 128
    cap_layers, min_bytes = 256, 1 << 30
    g = torch.Generator(device=dev)
    rows = []
    cfg = ext.TierConfig()
    cfg.promo_headroom_min = 8
    for B in args.cross_batches:
        for S in args.cross_contexts:
            g.manual_seed(args.seed + S + B)
            kv_bytes = 2 * B * Hkv * S * D * 2
            n_exact = max(1, min(cap_layers, -(-min_bytes // kv_bytes)))
            q = torch.randn((B, Hq, 1, D), generator=g, device=dev, dtype=torch.float32).half()
            kvs = [(torch.randn((B, Hkv, S, D), generator=g, device=dev, dtype=torch.float32).half(),
                    torch.randn((B, Hkv, S, D), generator=g, device=dev, dtype=torch.float32).half())
                   for _ in range(n_exact)]
            outs = torch.empty((B, Hq, 1, D), dtype=torch.float16, device=dev)
            qg = q.view(B, Hkv, Hq // Hkv, D).transpose(2, 3).contiguous()  # (B,Hkv,D,G)
            scale = D ** -0.5

            def sdpa_gqa(k, v):
                with sdpa_kernel(fused_backends):
                    outs.copy_(Fn.scaled_dot_product_attention(q, k, v, scale=scale, enable_gqa=True))

            def sdpa_ref(k, v):
                kk = k.repeat_interleave(Hq // Hkv, dim=1).contiguous()
                vv = v.repeat_interleave(Hq // Hkv, dim=1).contiguous()
                with sdpa_kernel(fused_backends):
                    outs.copy_(Fn.scaled_dot_product_attention(q, kk, vv, scale=scale))

            def gemm(k, v):
                sc = torch.matmul(k, qg).float() * scale                # (B,Hkv,S,G)
                p = torch.softmax(sc, dim=2).half().transpose(2, 3).contiguous()  # (B,Hkv,G,S)
                outs.copy_(torch.matmul(p, v).reshape(B, Hq, 1, D))

            exact = {}
            for name, fn in (("sdpa_gqa", sdpa_gqa), ("sdpa_repeat_interleave", sdpa_ref), ("fp16_gemm", gemm)):
                try:
                    ms = time_graph(torch, dev, [lambda kv=kv, fn=fn: fn(*kv) for kv in kvs], args.steps,
                                    args.warmup)
                    exact[name] = round(ms * 1e3 / n_exact, 3)
                except RuntimeError as e:  # a formulation torch cannot run here
                    exact[name] = f"unavailable: {str(e).splitlines()[0][:120]}"
                torch.cuda.synchronize()
            # fused: compress the first copy's tokens, replicate the blob per layer
            k0, v0 = kvs[0]
            cl = ext.CompressHandle(cfg).compress_layer(k0, v0, with_archive=False)
            del kvs
            torch.cuda.synchronize()
            handles, blob = [], 0
            while True:
                h = ext.FoveatedHandle(cl.near_k, cl.near_v, cl.far_k, cl.far_v, cl.far_v_scale, cl.far_v_zero,
                                       cl.near_valid, spike_margin=10.0)
                handles.append(h)
                blob += h.get_blob_info().blob_bytes
                if blob >= min_bytes or len(handles) >= cap_layers:
                    break
            res = [(torch.empty((B, Hq, 1, D), dtype=torch.float16, device=dev),
                    torch.empty((B, Hq), dtype=torch.int32, device=dev),
                    torch.empty((B, Hq), dtype=torch.int32, device=dev)) for _ in handles]
            ms = time_graph(torch, dev, [lambda h=h, r=r: h(q, out=r) for h, r in zip(handles, res)], args.steps,
                            args.warmup)
            fused_us = ms * 1e3 / len(handles)
            best = min(v for v in exact.values() if isinstance(v, float))
            row = {"B": B, "context": S, "exact_us": exact, "exact_best_us": best, "fused_us": round(fused_us, 3),
                   "speedup": round(best / fused_us, 3), "exact_layers": n_exact, "fused_layers": len(handles)}
            rows.append(row)
            print(f"[crossover] B={B} S={S}: exact {exact} fused {fused_us:.2f} us -> {best / fused_us:.2f}x",
                  file=sys.stderr, flush=True)
            del handles, res, cl
            torch.cuda.empty_cache()
    result = {
        "metric": "kernel crossover: fused two-tier attention vs exact fp16 attention, us/layer, 7B shapes, 1 GPU",
        "value": None, "unit": "us/layer", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "f16 operands, f32 accumulation", "data": "synthetic (seeded N(0,1) K, V, q)",
        "config": {"workload": "crossover_7b", "Hq": Hq, "Hkv": Hkv, "D": D, "near_pct": 0.10,
                   "far_format": "fp8-e4m3 K + int4 per-token V", "launch": "hip-graph, distinct layer copies"},
        "rows": rows,
    }
    if brief:
        return result
    print(json.dumps(result), flush=True)


def run_generate(args, torch, dev, brief=False):
    """The closure's host overhead against one HIP graph per model decode
    step: a seeded tiny LM (fp32 weights, --gen-layers layers of Hq=32,
    Hkv=8, D=128 attention, model dim 1024) prefills a --gen-context byte
    prompt, compresses, and decodes --gen-tokens greedy tokens through
    ``generate_fused`` three ways: the eager closure with the reference's
    host drain, the eager closure with the device drain, and the graph.
    Prints one JSON line: graph tokens/s as the value, host us per layer of
    each way (time spent issuing drain + model call, or the replay), and
    whether every way generated the same tokens."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    from _tiny_lm import ByteTokenizer, TinyLM

    from foveated_kv_amd import generate as gen

    L, n_tok, S = args.gen_layers, args.gen_tokens, args.gen_context
    model = TinyLM(vocab=256, dim=1024, n_layers=L, n_heads=32, n_kv_heads=8, head_dim=128, qk_gain=2.0,
                   seed=args.seed).to(dev).eval()
    tok = ByteTokenizer(vocab=256)
    rng = np.random.default_rng(args.seed)
    prompt = bytes(rng.integers(32, 127, size=S, dtype=np.uint8)).decode()
    print(f"[generate] tiny LM layers={L} Hq=32 Hkv=8 D=128 dim=1024 prompt={S} tokens={n_tok}",
          file=sys.stderr, flush=True)
    gen.generate_fused(model, tok, prompt[:256], max_tokens=4, enable_promotion=True, graph=True)  # warm
    torch.cuda.synchronize()
    runs = {}
    for name, kw in (("eager_host_drain", {}), ("eager_device_drain", {"device_drain": True}),
                     ("graph", {"graph": True})):
        text, st = gen.generate_fused(model, tok, prompt, max_tokens=n_tok, enable_promotion=True, **kw)
        runs[name] = (text, st)
        print(f"[generate] {name}: {st['tokens_per_second']:.1f} tok/s, host {st['host_us_per_layer']:.1f} "
              f"us/layer, promotions {st.get('promotions_completed')}", file=sys.stderr, flush=True)
    g = runs["graph"][1]
    keys = ("spikes_detected", "spikes_queued", "promotions_completed")
    result = {
        "metric": "tiny-LM greedy decode through the fused kernel, tokens/s (one HIP graph per decode step)",
        "value": round(g["tokens_per_second"], 2), "unit": "tokens/s", "n_gpus": 1, "steps": g["model_calls"],
        "warmup": 2, "ms_per_step": round(g["decode_time_s"] / max(g["model_calls"], 1) * 1e3, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "fp32 model, f16 attention operands", "data": "synthetic (seeded random weights and prompt)",
        "config": {"workload": "tiny_lm_generate", "layers": L, "Hq": 32, "Hkv": 8, "D": 128, "dim": 1024,
                   "prompt_tokens": S, "max_tokens": n_tok, "promotion": True, "qk_gain": 2.0},
        "ways": {n: {"tokens_per_second": round(st["tokens_per_second"], 2),
                     "host_us_per_layer": round(st["host_us_per_layer"], 2),
                     "closure_us_per_layer": (None if st["closure_us_per_layer"] is None
                                              else round(st["closure_us_per_layer"], 2)),
                     "decode_ms_per_token": round(st["decode_time_s"] / max(st["model_calls"], 1) * 1e3, 4),
                     **{k: st.get(k) for k in keys}} for n, (_, st) in runs.items()},
        "same_tokens": len({text for text, _ in runs.values()}) == 1,
        "same_promotions": len({tuple(st.get(k) for k in keys) for _, st in runs.values()}) == 1,
    }
    if brief:
        return result
    print(json.dumps(result), flush=True)


def copy_bandwidth(torch, dev, mib, reps=20):
    """Read + write GB/s of a plain device-to-device tensor copy of ``mib`` MiB
    (the calibration kernel for HBM counters and the practical copy ceiling)."""
    n = mib * (1 << 20)
    src = torch.empty(n, dtype=torch.uint8, device=dev).fill_(1)
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(reps):
        dst.copy_(src)
    end.record()
    torch.cuda.synchronize()
    sec = start.elapsed_time(end) / 1e3 / reps
    print(f"[bench] copy of {mib} MiB: {sec * 1e6:.1f} us -> {2 * n / sec / 1e9:.1f} GB/s (read + write)",
          file=sys.stderr, flush=True)
    return round(2 * n / sec / 1e9, 1)


def read_ceiling(torch, dev, mib, reps=20, sweep=True):
    """Best read GB/s of the library's streaming-read probe over ``mib`` MiB,
    swept over loads in flight per lane, non-temporal hint and grid size
    (``sweep=False``: only the best launch found on MI355X)."""
    from foveated_kv_amd import _lib

    lib = _lib.load()
    n = mib * (1 << 20)
    buf = torch.empty(n, dtype=torch.uint8, device=dev).fill_(3)
    best = (0.0, None)
    for blocks in ((1024, 2048, 4096, 8192) if sweep else (2048,)):
        out = torch.empty(blocks * 4, dtype=torch.int32, device=dev)
        for unroll in ((1, 2, 4, 8) if sweep else (1,)):
            for nt in ((0, 1) if sweep else (1,)):
                def run():
                    _lib.check(lib.fkv_hbm_read_probe(_lib.ptr(buf), n, unroll, nt, blocks, _lib.ptr(out),
                                                      _lib.stream_ptr(dev)), "fkv_hbm_read_probe")
                run()
                torch.cuda.synchronize()
                start = torch.cuda.Event(enable_timing=True)
                end = torch.cuda.Event(enable_timing=True)
                start.record()
                for _ in range(reps):
                    run()
                end.record()
                torch.cuda.synchronize()
                gbs = n / (start.elapsed_time(end) / 1e3 / reps) / 1e9
                print(f"[bench] read probe blocks={blocks} unroll={unroll} nt={nt}: {gbs:.1f} GB/s",
                      file=sys.stderr, flush=True)
                if gbs > best[0]:
                    best = (gbs, dict(blocks=blocks, unroll=unroll, nontemporal=nt))
    return round(best[0], 1), best[1]


if __name__ == "__main__":
    main()
