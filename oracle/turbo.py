"""CPU restatement of the TurboQuant far tier -- TEST INFRASTRUCTURE ONLY.

Restates samfurr/foveated_kv src/foveated_kv/turbo_constants.py:29-100
(constants), turbo_quantize.py:25-313 (compress / dequant / score) and,
through ``orc_attend_turbo`` in fkv_oracle.c, the fused turbo kernel
(csrc/kernels/foveated_attn.metal:486-767, host q prep
csrc/foveated_attn.cpp:407-491).  Only ``tests/`` (and the fixture script
under ``tests/golden/``) may import it; the product package never does.

Arithmetic: the reference runs these in MLX fp32.  Here compression is
evaluated in fp64 from the same fp32/fp16 inputs (the more exact value of
the same formula); the tests compare the GPU's fp32 results against it with
the decision margins exposed (``compress_keys(..., margins=True)``), so a
code that sits within rounding of a Lloyd-Max boundary or of a QJL sign
change is not counted as a mismatch.  Value compression is elementwise and
restated in fp32 op order (bit-exact target).

Pinning (tests/test_oracle_turbo.py): constants by QR uniqueness,
orthogonality, the RandomState stream and the textbook 2-bit Lloyd-Max
quantiser (Max 1960); compress by planted keys whose codes are known by
construction and by the dequantisation relations (stage-1 reconstruction,
residual norm, QJL sketch direction); value codes by closed forms and
half-to-even ties; the kernel's score by the dequantised-key identities;
attention by brute force and split-count invariance.
"""

import ctypes
import math

import numpy as np

from . import _load, _ptr, _u16

# ---------------------------------------------------------------------------
# constants (turbo_constants.py:29-100)
# ---------------------------------------------------------------------------


def rotation_matrix(d, seed=42):
    """turbo_constants.py:43-53: Q of the QR factorisation of a seeded fp32
    Gaussian matrix, columns sign-fixed so that diag(R) > 0."""
    h = np.random.RandomState(seed).randn(d, d).astype(np.float32)
    q, r = np.linalg.qr(h)
    s = np.sign(np.diag(r))
    s[s == 0] = 1
    return (q * s[np.newaxis, :]).astype(np.float32)


def qjl_matrix(d, seed=137):
    """turbo_constants.py:56-59.  Under NumPy >= 2 the fp32 Gaussian is
    divided by a float64 scalar in float64, then stored as fp32."""
    g = np.random.RandomState(seed).randn(d, d).astype(np.float32)
    return (g.astype(np.float64) / np.sqrt(d)).astype(np.float32)


def lloyd_max(d, bits=2, n_iters=200):
    """turbo_constants.py:62-100: Lloyd-Max on N(0, 1/d) from the
    N-quantile initial boundaries, conditional means by the Gaussian closed
    form; returns fp32 (centroids, boundaries)."""
    from scipy.stats import norm

    n = 2 ** bits
    sigma = 1.0 / np.sqrt(d)
    b = norm.ppf(np.linspace(0, 1, n + 1)[1:-1], scale=sigma)
    for _ in range(n_iters):
        ext = np.concatenate([[-np.inf], b, [np.inf]])
        c = np.zeros(n)
        for i in range(n):
            lo, hi = ext[i], ext[i + 1]
            prob = norm.cdf(hi, scale=sigma) - norm.cdf(lo, scale=sigma)
            if prob > 1e-15:
                c[i] = sigma ** 2 * (norm.pdf(lo, scale=sigma) - norm.pdf(hi, scale=sigma)) / prob
            else:
                c[i] = (lo + hi) / 2 if np.isfinite(lo + hi) else 0
        b = (c[:-1] + c[1:]) / 2
    return c.astype(np.float32), b.astype(np.float32)


def constants(d, pi_seed=42, s_seed=137):
    c, b = lloyd_max(d)
    return {"Pi": rotation_matrix(d, pi_seed), "S": qjl_matrix(d, s_seed), "centroids": c, "boundaries": b}


# ---------------------------------------------------------------------------
# bit packing (turbo_quantize.py:66-83, 282-313)
# ---------------------------------------------------------------------------


def pack_2bit(codes):
    c = np.asarray(codes, np.uint8)
    r = c.reshape(c.shape[:-1] + (c.shape[-1] // 4, 4))
    return (r[..., 0] | (r[..., 1] << 2) | (r[..., 2] << 4) | (r[..., 3] << 6)).astype(np.uint8)


def unpack_2bit(packed):
    p = np.asarray(packed, np.uint8)
    out = np.stack([(p >> (2 * i)) & 3 for i in range(4)], axis=-1)
    return out.reshape(p.shape[:-1] + (p.shape[-1] * 4,)).astype(np.uint8)


def pack_1bit(bits):
    b = np.asarray(bits, np.uint8)
    r = b.reshape(b.shape[:-1] + (b.shape[-1] // 8, 8))
    out = np.zeros(r.shape[:-1], np.uint8)
    for i in range(8):
        out |= (r[..., i] & 1) << i
    return out


def unpack_1bit(packed):
    """-> +-1 float64 (bit 1 -> +1)."""
    p = np.asarray(packed, np.uint8)
    bits = np.stack([(p >> i) & 1 for i in range(8)], axis=-1)
    bits = bits.reshape(p.shape[:-1] + (p.shape[-1] * 8,))
    return 2.0 * bits.astype(np.float64) - 1.0


# ---------------------------------------------------------------------------
# compression (turbo_quantize.py:25-91, 139-178)
# ---------------------------------------------------------------------------


def compress_keys(keys, C, margins=False):
    """turbo_compress_keys on (B,H,N,D) fp16 keys -> (idx u8 (..,D/4), signs
    u8 (..,D/8), norm fp16, gamma fp16); with ``margins`` also the distance
    of every rotated coordinate to its nearest boundary and |S r| per dim
    (fp64), the decisions a rounding change could flip."""
    k = np.asarray(keys, np.float16).astype(np.float64)
    Pi = C["Pi"].astype(np.float64)
    S = C["S"].astype(np.float64)
    cb = C["centroids"].astype(np.float64)
    bd = C["boundaries"].astype(np.float64)
    norm = np.sqrt((k * k).sum(-1))
    y = (k / np.maximum(norm, 1e-8)[..., None]) @ Pi.T
    idx = ((y >= bd[0]).astype(np.uint8) + (y >= bd[1]) + (y >= bd[2])).astype(np.uint8)
    k_hat = norm[..., None] * (cb[idx] @ Pi)
    r = k - k_hat
    gamma = np.sqrt((r * r).sum(-1))
    proj = r @ S.T
    signs = (proj >= 0).astype(np.uint8)
    out = (pack_2bit(idx), pack_1bit(signs), norm.astype(np.float16), gamma.astype(np.float16))
    if margins:
        ymarg = np.min(np.abs(y[..., None] - bd), axis=-1)
        return out + (ymarg, np.abs(proj), idx, signs)
    return out


def compress_values(values, group=32):
    """turbo_compress_values in fp32 op order: per 32-dim group scale =
    max(max|v|, 1e-8); code = clip(round_half_even((v/scale + 1) * 1.5),
    0, 3); scale stored as fp16."""
    v = np.asarray(values, np.float16).astype(np.float32)
    sh = v.shape
    g = v.reshape(sh[:-1] + (sh[-1] // group, group))
    scale = np.maximum(np.max(np.abs(g), axis=-1), np.float32(1e-8)).astype(np.float32)
    x = g / scale[..., None]
    x = (x + np.float32(1.0)).astype(np.float32)
    x = (x * np.float32(1.5)).astype(np.float32)
    codes = np.clip(np.rint(x), 0, 3).astype(np.uint8).reshape(sh)
    return pack_2bit(codes), scale.astype(np.float16)


VAL_LEVELS = np.array([-1.0, -1.0 / 3.0, 1.0 / 3.0, 1.0], np.float32)  # turbo_quantize.py:16
KERNEL_LEVELS = np.array([-1.0, -0.333333, 0.333333, 1.0], np.float32)  # foveated_attn.metal:529


def dequant_keys(idx, signs, norm, gamma, C, as_f16=True):
    """turbo_dequant_keys (turbo_quantize.py:94-133): norm * (cb[idx] @ Pi) +
    gamma * (signs @ S) / D, as fp16 (evaluated in fp64; ``as_f16=False``
    returns the fp64 value before the final cast)."""
    codes = unpack_2bit(idx)
    D = codes.shape[-1]
    k_mse = np.asarray(norm, np.float16).astype(np.float64)[..., None] * (
        C["centroids"].astype(np.float64)[codes] @ C["Pi"].astype(np.float64))
    r_hat = np.asarray(gamma, np.float16).astype(np.float64)[..., None] * (
        unpack_1bit(signs) @ C["S"].astype(np.float64)) / D
    k = k_mse + r_hat
    return k.astype(np.float16) if as_f16 else k


def dequant_values(packed, scales, group=32):
    """turbo_dequant_values (turbo_quantize.py:181-206) -> fp16."""
    codes = unpack_2bit(packed)
    lv = VAL_LEVELS[codes].astype(np.float32)
    sh = lv.shape
    g = lv.reshape(sh[:-1] + (sh[-1] // group, group))
    return (g * np.asarray(scales, np.float16).astype(np.float32)[..., None]).reshape(sh).astype(np.float16)


def score_keys(query, idx, signs, norm, gamma, C):
    """turbo_score_keys (turbo_quantize.py:213-279): GQA groups averaged in
    the rotated / sketched domain; -> (B, H_kv, N) fp64."""
    q = np.asarray(query, np.float16).astype(np.float64)
    if q.ndim == 4:
        q = q[:, :, 0, :]
    codes = unpack_2bit(idx)
    B, Hkv, N, D = codes.shape
    q_rot = q @ C["Pi"].astype(np.float64).T
    q_sk = q @ C["S"].astype(np.float64).T
    if q.shape[1] != Hkv:
        g = q.shape[1] // Hkv
        q_rot = q_rot.reshape(B, Hkv, g, D).mean(2)
        q_sk = q_sk.reshape(B, Hkv, g, D).mean(2)
    mse = np.asarray(norm, np.float16).astype(np.float64) * np.einsum(
        "bhd,bhnd->bhn", q_rot, C["centroids"].astype(np.float64)[codes])
    sd = np.einsum("bhd,bhnd->bhn", q_sk, unpack_1bit(signs))
    return mse + (math.sqrt(math.pi / 2) / D) * np.asarray(gamma, np.float16).astype(np.float64) * sd


# ---------------------------------------------------------------------------
# fused kernel (foveated_attn.metal:559-767) and the formulation
# ---------------------------------------------------------------------------


def qprep(q, C):
    """foveated_attn.cpp:415-421: q cast to fp16, then q.Pi^T and q.S^T."""
    q16 = np.asarray(q, np.float16)
    B, Hq = q16.shape[:2]
    D = q16.shape[-1]
    qf = q16.reshape(B, Hq, D).astype(np.float64)
    return qf @ C["Pi"].astype(np.float64).T, qf @ C["S"].astype(np.float64).T


def far_scores(q, k_idx, k_signs, k_norm, k_gamma, C):
    """Per q head far-token scores of the fused kernel (dot_turbo_k,
    foveated_attn.metal:486-521, times rsqrt(D) at :700-704), fp64:
    (norm * q_rot.cb[idx] + (1.2533141/D) * gamma * q_sketch.signs) / sqrt(D).
    -> (B, Hq, F); GQA maps q head h to kv head h // (Hq/Hkv)."""
    q_rot, q_sk = qprep(q, C)
    codes = unpack_2bit(k_idx)
    B, Hkv, F, D = codes.shape
    Hq = q_rot.shape[1]
    g = Hq // Hkv
    cbv = C["centroids"].astype(np.float64)[codes]  # (B,Hkv,F,D)
    sg = unpack_1bit(k_signs)
    cbv = np.repeat(cbv, g, axis=1)
    sg = np.repeat(sg, g, axis=1)
    nrm = np.repeat(np.asarray(k_norm, np.float16).astype(np.float64), g, axis=1)
    gam = np.repeat(np.asarray(k_gamma, np.float16).astype(np.float64), g, axis=1)
    mse = np.einsum("bhd,bhfd->bhf", q_rot, cbv)
    sd = np.einsum("bhd,bhfd->bhf", q_sk, sg)
    qjl = float(np.float32(1.2533141) / np.float32(D))
    inv = float(np.float32(1.0) / np.sqrt(np.float32(D)))
    return (nrm * mse + qjl * gam * sd) * inv


def far_values(v_packed, v_scale):
    """load_turbo_v (foveated_attn.metal:531-552): level[code] * scale, fp64."""
    codes = unpack_2bit(v_packed)
    sh = codes.shape
    lv = KERNEL_LEVELS.astype(np.float64)[codes].reshape(sh[:-1] + (sh[-1] // 32, 32))
    sc = np.asarray(v_scale, np.float16).astype(np.float64)[..., None]
    return (lv * sc).reshape(sh)


def attend_kernel(q, near_k, near_v, near_valid, k_idx, k_signs, k_norm, k_gamma, v_packed, v_scale, C,
                  dec_k=None, dec_v=None, spike_margin=10.0, split_size=0, num_splits=0, gate=True):
    """Fused turbo kernel semantics in fp64 (orc_attend_turbo).  Returns
    (out (B,Hq,D), flags, tokens, max_far, min_near)."""
    lib = _load()
    fn = lib.orc_attend_turbo
    P, I = ctypes.c_void_p, ctypes.c_int
    fn.restype = I
    fn.argtypes = [I] * 7 + [P] * 15 + [ctypes.c_float, I, I, I] + [P] * 5
    q16 = np.ascontiguousarray(np.asarray(q, np.float16))
    B, Hq = q16.shape[:2]
    D = q16.shape[-1]
    q16 = q16.reshape(B, Hq, D)
    q_rot, q_sk = qprep(q16, C)
    nk, nv_ = _u16(near_k), _u16(near_v)
    Hkv, Npad = nk.shape[1], nk.shape[2]
    ki = np.ascontiguousarray(k_idx, np.uint8)
    F = ki.shape[2]
    ks = np.ascontiguousarray(k_signs, np.uint8)
    kn, kg = _u16(np.asarray(k_norm, np.float16)), _u16(np.asarray(k_gamma, np.float16))
    vp = np.ascontiguousarray(v_packed, np.uint8)
    vs = _u16(np.asarray(v_scale, np.float16))
    cb = np.ascontiguousarray(C["centroids"], np.float32)
    if dec_k is None:
        dk = dv = np.zeros((B, Hkv, 0, D), np.uint16)
        ndec = 0
    else:
        dk, dv, ndec = _u16(dec_k), _u16(dec_v), dec_k.shape[2]
    valid = np.ascontiguousarray(near_valid, np.uint32)
    out = np.zeros((B, Hq, D), np.float64)
    flags = np.zeros((B, Hq), np.int32)
    tokens = np.zeros((B, Hq), np.int32)
    mf = np.zeros((B, Hq), np.float64)
    mn = np.zeros((B, Hq), np.float64)
    rc = fn(B, Hq, Hkv, D, Npad, F, ndec, _ptr(q16.view(np.uint16)), _ptr(np.ascontiguousarray(q_rot)),
            _ptr(np.ascontiguousarray(q_sk)), _ptr(nk), _ptr(nv_), _ptr(valid), _ptr(ki), _ptr(ks), _ptr(kn),
            _ptr(kg), _ptr(vp), _ptr(vs), _ptr(cb), _ptr(dk), _ptr(dv), float(spike_margin), int(split_size),
            int(num_splits), int(bool(gate)), _ptr(out), _ptr(flags), _ptr(tokens), _ptr(mf), _ptr(mn))
    if rc != 0:
        raise ValueError(f"orc_attend_turbo failed: {rc}")
    return out, flags, tokens, mf, mn


def attend_formulation(q, near_k, near_v, near_valid, k_idx, k_signs, k_norm, k_gamma, v_packed, v_scale, C,
                       dec_k=None, dec_v=None):
    """MLXFoveatedLayer._attend_turbo (mlx_foveated.py:280-312): dequantised
    far keys / values (fp16) after near[:max(near_valid)] ++ decode, SDPA
    with scale D^-1/2 in fp64, GQA by repeat."""
    q = np.asarray(q, np.float16).astype(np.float64)
    B, Hq = q.shape[:2]
    D = q.shape[-1]
    q = q.reshape(B, Hq, D)
    nk = np.asarray(near_k, np.float16)
    nv_ = np.asarray(near_v, np.float16)
    Hkv = nk.shape[1]
    mv = int(np.max(near_valid))
    ks = [nk[:, :, :mv]]
    vs = [nv_[:, :, :mv]]
    if dec_k is not None:
        ks.append(np.asarray(dec_k, np.float16))
        vs.append(np.asarray(dec_v, np.float16))
    ks.append(dequant_keys(k_idx, k_signs, k_norm, k_gamma, C))
    vs.append(dequant_values(v_packed, v_scale))
    K = np.concatenate(ks, axis=2).astype(np.float64)
    V = np.concatenate(vs, axis=2).astype(np.float64)
    g = Hq // Hkv
    K = np.repeat(K, g, axis=1)
    V = np.repeat(V, g, axis=1)
    s = np.einsum("bhd,bhnd->bhn", q, K) / math.sqrt(D)
    s = s - s.max(-1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(-1, keepdims=True)
    return np.einsum("bhn,bhnd->bhd", p, V)
