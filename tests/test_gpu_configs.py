"""GPU parity at the benchmark configurations' full shapes.

C3 (7B shapes, batch 8, 16K and 32K context, fp8 K with per-token or
group-32 INT4 V, 2 % of far tokens planted above the near-tier minimum) and
C4 (TurboQuant, batch 4, 8K context) run through the C ABI exactly as the
benchmark launches them, and are checked against the CPU oracle on the same
compressed inputs: outputs within max-abs 2e-3 and cosine 0.9999 of the
kernel restatement (and, for C3, of the reference's dequant + SDPA
formulation), spike flags and tokens equal except on exact-score ties.  The
C5 loop at its full shape is in test_gpu_e2e.py.
"""

import numpy as np
import pytest
import torch

from _parity import ATOL, COS, flush, np_, record, run_attention

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def fkv():
    import foveated_kv_amd
    from foveated_kv_amd import _lib

    _lib.load()
    assert torch.cuda.is_available(), "GPU tests need a ROCm device"
    assert foveated_kv_amd.is_available(), "libfkv.so loaded but no gfx950 device"
    return foveated_kv_amd


C3 = [(16384, 0), (16384, 32), (32768, 0), (32768, 32), (8192, 32)]


@pytest.mark.parametrize("S,vg", C3, ids=[f"{s // 1024}k_{'g32' if g else 'per_token'}" for s, g in C3])
def test_c3_full_shape(fkv, orc, S, vg):
    """C3: B=8, Hq=32, Hkv=8, D=128, 2 % planted spikes (the 8K per-token
    case is test_gpu_parity.py::test_attention_config3_8k)."""
    _, flags, _, kf = run_attention(fkv, orc, 8, 32, 8, 128, S, 0, seed=100 + S // 1024 + vg, spikes=0.02,
                                    v_group=vg)
    assert kf.sum() > 0 and flags.sum() > 0  # the planted tokens are flagged


def test_c4_turbo_full_shape(fkv, orc):
    """C4: TurboQuant far tier at B=4, Hq=32, Hkv=8, D=128, 8K context,
    built the way the benchmark builds it (fused compress, then GPU
    TurboQuant compression of the archived far rows), against the kernel
    restatement on the GPU's own codes."""
    from oracle import turbo as T

    from foveated_kv_amd import ext, synthetic
    from foveated_kv_amd import turbo as tq

    B, Hq, Hkv, D, S = 4, 32, 8, 128, 8192
    seed = 400
    case = f"C4 turbo B={B} Hq={Hq} Hkv={Hkv} D={D} S={S} spikes=0.02"
    flush(case)
    cfg = ext.TierConfig()
    cfg.promo_headroom_min = 8
    tb = ext.tier_boundaries_c(cfg, S)
    k, v = synthetic.make_kv(B, Hkv, S, D, seed)
    q = synthetic.make_query(B, Hq, D, seed)
    synthetic.inject_spikes(k, q, tb["mid_start"], tb["far_count"], 0.02, seed)
    cl = ext.CompressHandle(cfg).compress_layer(torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda(),
                                                with_archive=True)
    del k, v
    tc = tq.get_turbo_constants(D)
    far = tq.turbo_compress_keys(cl.archive_k, tc) + tq.turbo_compress_values(cl.archive_v)
    h = tq.TurboFoveatedHandle(cl.near_k, cl.near_v, *far, cl.near_valid, tc.Pi, tc.S, tc.centroids,
                               spike_margin=10.0)
    qt = torch.from_numpy(q).cuda()
    out, flags, toks = h(qt[:, :, None, :])
    torch.cuda.synchronize()
    out = np_(out)[:, :, 0].astype(np.float64)
    flags, toks = np_(flags), np_(toks)
    C = T.constants(D)
    L = dict(near_k=np_(cl.near_k), near_v=np_(cl.near_v), near_valid=np_(cl.near_valid).astype(np.uint32),
             k_idx=np_(far[0]), k_signs=np_(far[1]), k_norm=np_(far[2]), k_gamma=np_(far[3]),
             v_packed=np_(far[4]), v_scale=np_(far[5]))
    ko, kf, kt, mf, mn = T.attend_kernel(q, **L, C=C, spike_margin=10.0)
    err = float(np.abs(out - ko).max())
    cos = orc.cosine(out, ko)
    flush(f"  vs kernel restatement: max-abs {err:.3e} cos {cos:.8f}")
    assert err <= ATOL and cos >= COS
    ties = 0
    fs = None
    for b, hh in np.argwhere(toks != kt):
        if fs is None:
            fs = T.far_scores(q, L["k_idx"], L["k_signs"], L["k_norm"], L["k_gamma"], C)
        assert abs(fs[b, hh, toks[b, hh]] - fs[b, hh, kt[b, hh]]) < 1e-3, (b, hh)
        ties += 1
    for b, hh in np.argwhere(flags != kf):
        assert abs(mf[b, hh] - (mn[b, hh] + 10.0)) < 1e-3, (b, hh)
        ties += 1
    assert kf.sum() > 0 and flags.sum() > 0
    record(case, maxabs_kernel=err, cos_kernel=cos, flagged=int(flags.sum()), spike_ties=ties)
