"""Seeded synthetic decode workloads for the benchmark configurations.

K, V ~ N(0,1) fp16 with a few outlier channels, q ~ N(0,1), an optional
fraction of far tokens aligned with the group's query direction so their
scores clear the spike margin (exercises spike detection and the V gate).
Everything is generated with numpy from a seed, so CPU checkers and the GPU
path see identical inputs.
"""

import numpy as np

CONFIGS = {
    # name: (B, Hq, Hkv, D, S, n_dec)
    "c1_qwen05b_512": (1, 14, 2, 64, 512, 16),
    "c2_7b_4k": (1, 32, 8, 128, 4096, 64),
    "c3_7b_8k_b8": (8, 32, 8, 128, 8192, 0),
    "c3_7b_16k_b8": (8, 32, 8, 128, 16384, 0),
    "c3_7b_32k_b8": (8, 32, 8, 128, 32768, 0),
    "c4_turbo_8k_b4": (4, 32, 8, 128, 8192, 0),
    "c5_70b_64k": (1, 64, 8, 128, 65536, 0),
}


def make_kv(B, H, S, D, seed, n_outlier=4, outlier_scale=8.0, heavy_tail=False):
    rng = np.random.default_rng(seed)
    k = rng.standard_normal((B, H, S, D), dtype=np.float32)
    v = rng.standard_normal((B, H, S, D), dtype=np.float32)
    if n_outlier:
        ch = rng.choice(D, size=n_outlier, replace=False)
        if heavy_tail:
            # per-channel Student-t(3) scale around the outlier factor
            sc = outlier_scale * np.abs(rng.standard_t(3, size=n_outlier)).clip(0.5, 4.0)
        else:
            sc = np.full(n_outlier, outlier_scale)
        k[..., ch] *= sc.astype(np.float32)
    return k.astype(np.float16), v.astype(np.float16)


def make_query(B, Hq, D, seed):
    rng = np.random.default_rng(seed + 1)
    return rng.standard_normal((B, Hq, D), dtype=np.float32).astype(np.float16)


def inject_spikes(keys, q, far_start, far_count, frac, seed, score=14.0):
    """Overwrite ``frac`` of the far positions of every (b, kv head) with
    k = alpha * unit(mean query of the group) + small noise, alpha chosen so
    that the group's mean-query score is ``score`` (well above the near-tier
    minimum + the 10.0 margin for N(0,1) data).  Returns the positions."""
    if frac <= 0 or far_count <= 0:
        return np.zeros((keys.shape[0], keys.shape[1], 0), np.int64)
    rng = np.random.default_rng(seed + 2)
    B, Hkv, S, D = keys.shape
    G = q.shape[1] // Hkv
    n = max(1, int(far_count * frac))
    pos = np.zeros((B, Hkv, n), np.int64)
    for b in range(B):
        for h in range(Hkv):
            qm = q[b, h * G:(h + 1) * G].astype(np.float32).mean(0)
            u = qm / (np.linalg.norm(qm) + 1e-6)
            alpha = score * np.sqrt(D) / (np.linalg.norm(qm) + 1e-6)
            p = far_start + rng.choice(far_count, size=n, replace=False)
            noise = 0.05 * rng.standard_normal((n, D), dtype=np.float32)
            keys[b, h, p] = (alpha * u[None] + noise).astype(np.float16)
            pos[b, h] = np.sort(p)
    return pos


def inject_spikes_at(keys, q, far_idx, frac, seed, score=14.0):
    """inject_spikes for a scattered far tier: ``far_idx`` (B, Hkv, F) holds
    the far positions of each (b, kv head) (an importance partition)."""
    if frac <= 0 or far_idx.shape[2] == 0:
        return np.zeros(far_idx.shape[:2] + (0,), np.int64)
    rng = np.random.default_rng(seed + 2)
    B, Hkv, S, D = keys.shape
    G = q.shape[1] // Hkv
    F = far_idx.shape[2]
    n = max(1, int(F * frac))
    pos = np.zeros((B, Hkv, n), np.int64)
    for b in range(B):
        for h in range(Hkv):
            qm = q[b, h * G:(h + 1) * G].astype(np.float32).mean(0)
            u = qm / (np.linalg.norm(qm) + 1e-6)
            alpha = score * np.sqrt(D) / (np.linalg.norm(qm) + 1e-6)
            p = np.asarray(far_idx[b, h])[rng.choice(F, size=n, replace=False)]
            noise = 0.05 * rng.standard_normal((n, D), dtype=np.float32)
            keys[b, h, p] = (alpha * u[None] + noise).astype(np.float16)
            pos[b, h] = np.sort(p)
    return pos


def make_importance(B, H, S, seed):
    """Seeded importance scores (B, H, S) fp32 for the importance partition."""
    rng = np.random.default_rng(seed + 4)
    return rng.standard_normal((B, H, S), dtype=np.float32)


def drift_queries(q0, steps, eps, seed):
    """Per-step query drift q_t = |q_0| * unit(q_{t-1} + eps * |q_0| * u_t),
    u_t ~ N(0, I/D) per head: (steps, B, Hq, D) fp16."""
    rng = np.random.default_rng(seed + 5)
    q = q0.astype(np.float32)
    norm = np.linalg.norm(q, axis=-1, keepdims=True)
    D = q.shape[-1]
    out = np.empty((steps,) + q.shape, np.float16)
    for t in range(steps):
        u = rng.standard_normal(q.shape, dtype=np.float32) / np.sqrt(D)
        q = q + eps * norm * u
        q = q / (np.linalg.norm(q, axis=-1, keepdims=True) + 1e-12) * norm
        out[t] = q.astype(np.float16)
    return out


def make_decode(B, Hkv, n_dec, D, seed):
    if n_dec == 0:
        return None, None
    rng = np.random.default_rng(seed + 3)
    dk = rng.standard_normal((B, Hkv, n_dec, D), dtype=np.float32).astype(np.float16)
    dv = rng.standard_normal((B, Hkv, n_dec, D), dtype=np.float32).astype(np.float16)
    return dk, dv
