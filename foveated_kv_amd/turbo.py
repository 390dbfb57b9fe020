"""TurboQuant far tier on the gfx950 library.

Mirrors samfurr/foveated_kv:
  get_turbo_constants / TurboConstants   turbo_constants.py:19-100
  turbo_compress_keys / _values          turbo_quantize.py:25-91, 139-178  (HIP kernels)
  turbo_dequant_keys / _values           turbo_quantize.py:94-133, 181-206 (torch ops)
  turbo_score_keys                       turbo_quantize.py:213-279          (torch ops)
  TurboFoveatedHandle                    csrc/foveated_attn.cpp:365-491     (HIP kernel)
  build_turbo_layer                      mlx_foveated.py:799-944 (turbo branch)

Compression and the fused attention run on the GPU through libfkv.so; the
dequantisation / score functions are the reference's formulation in torch
ops (the path ``FoveatedLayer.attend`` uses).  The kernel keeps the
reference kernel's QJL factor sqrt(pi/2)/D and value levels
{-1, -0.333333, 0.333333, 1}; the dequantisation keeps the reference's 1/D
and {-1, -1/3, 1/3, 1} -- the two reference paths differ by design.
"""

import ctypes
import math
from dataclasses import dataclass
from functools import lru_cache
from statistics import NormalDist

import numpy as np
import torch

from . import _lib, ext
from ._lib import check, dtype_code, ptr

# ---------------------------------------------------------------------------
# constants (turbo_constants.py:19-100)
# ---------------------------------------------------------------------------


@dataclass(frozen=True)
class TurboConstants:
    """Pi (D,D) rotation, S (D,D) QJL matrix, Lloyd-Max centroids (4,) and
    boundaries (3,), fp32 CPU tensors; ``on(device)`` returns device copies
    (cached)."""

    Pi: torch.Tensor
    S: torch.Tensor
    centroids: torch.Tensor
    boundaries: torch.Tensor

    def on(self, device):
        return _constants_on(self, torch.device(device))


_device_cache = {}


def _constants_on(tc, device):
    key = (id(tc), str(device))
    hit = _device_cache.get(key)
    if hit is None:
        hit = TurboConstants(tc.Pi.to(device), tc.S.to(device), tc.centroids.to(device), tc.boundaries.to(device))
        _device_cache[key] = hit
    return hit


def _rotation_matrix(d, seed):
    """Q of the QR factorisation of a seeded fp32 Gaussian matrix with
    diag(R) > 0 (turbo_constants.py:43-53)."""
    h = np.random.RandomState(seed).randn(d, d).astype(np.float32)
    q, r = np.linalg.qr(h)
    s = np.sign(np.diag(r))
    s[s == 0] = 1
    return (q * s[np.newaxis, :]).astype(np.float32)


def _qjl_matrix(d, seed):
    """turbo_constants.py:56-59 (fp32 Gaussian / sqrt(d), divided in fp64)."""
    g = np.random.RandomState(seed).randn(d, d).astype(np.float32)
    return (g.astype(np.float64) / np.sqrt(d)).astype(np.float32)


def _normal(sigma):
    """(ppf, pdf, cdf) of N(0, sigma^2): scipy.stats.norm as the reference
    uses, else the standard library (equal to ~1e-16; the boundary between
    the two inner cells is then 0 to within ~1e-17 either way)."""
    try:
        from scipy.stats import norm

        return (lambda q: float(norm.ppf(q, scale=sigma)), lambda x: float(norm.pdf(x, scale=sigma)),
                lambda x: float(norm.cdf(x, scale=sigma)))
    except ImportError:
        nd = NormalDist(0.0, sigma)
        return nd.inv_cdf, nd.pdf, nd.cdf


def _lloyd_max(d, bits=2, n_iters=200):
    """Lloyd-Max on N(0, 1/d) from the quantile boundaries, 200 iterations
    (turbo_constants.py:62-100)."""
    n = 2 ** bits
    sigma = 1.0 / math.sqrt(d)
    ppf, pdf, cdf = _normal(sigma)
    b = [ppf(q) for q in np.linspace(0, 1, n + 1)[1:-1]]
    c = [0.0] * n
    for _ in range(n_iters):
        ext_ = [-math.inf] + list(b) + [math.inf]
        for i in range(n):
            lo, hi = ext_[i], ext_[i + 1]
            prob = cdf(hi) - cdf(lo)
            if prob > 1e-15:
                c[i] = sigma ** 2 * (pdf(lo) - pdf(hi)) / prob
            else:
                c[i] = (lo + hi) / 2 if math.isfinite(lo + hi) else 0.0
        b = [(c[i] + c[i + 1]) / 2 for i in range(n - 1)]
    return np.asarray(c, np.float32), np.asarray(b, np.float32)


@lru_cache(maxsize=4)
def get_turbo_constants(d: int, pi_seed: int = 42, s_seed: int = 137) -> TurboConstants:
    c, b = _lloyd_max(d)
    return TurboConstants(Pi=torch.from_numpy(_rotation_matrix(d, pi_seed)),
                          S=torch.from_numpy(_qjl_matrix(d, s_seed)),
                          centroids=torch.from_numpy(c), boundaries=torch.from_numpy(b))


# ---------------------------------------------------------------------------
# compression (HIP kernels)
# ---------------------------------------------------------------------------


def _f32(t, device):
    return t.to(device=device, dtype=torch.float32).contiguous()


def turbo_compress_keys(keys: torch.Tensor, tc: TurboConstants):
    """(B,H,N,D) keys -> indices (B,H,N,D/4) u8, signs (B,H,N,D/8) u8,
    norms (B,H,N) fp16, gamma (B,H,N) fp16 (turbo_quantize.py:25-91)."""
    ext._require_device(keys)
    B, H, N, D = keys.shape
    dev = keys.device
    k = keys if keys.dtype in (torch.float16, torch.bfloat16, torch.float32) else keys.half()
    k = k.contiguous()
    idx = torch.empty((B, H, N, D // 4), dtype=torch.uint8, device=dev)
    sgn = torch.empty((B, H, N, D // 8), dtype=torch.uint8, device=dev)
    nrm = torch.empty((B, H, N), dtype=torch.float16, device=dev)
    gam = torch.empty_like(nrm)
    if k.numel() == 0:
        return idx, sgn, nrm, gam
    c = tc.on(dev)
    lib = _lib.load()
    with torch.cuda.device(dev):
        check(lib.fkv_turbo_compress_keys(ptr(k), dtype_code(k.dtype), B * H * N, D, ptr(_f32(c.Pi, dev)),
                                          ptr(_f32(c.S, dev)), ptr(_f32(c.centroids, dev)),
                                          ptr(_f32(c.boundaries, dev)), ptr(idx), ptr(sgn), ptr(nrm), ptr(gam),
                                          _lib.stream_ptr(dev)), "fkv_turbo_compress_keys")
    return idx, sgn, nrm, gam


def turbo_compress_values(values: torch.Tensor, group_size: int = 32):
    """(B,H,N,D) values -> packed (B,H,N,D/4) u8, scales (B,H,N,D/32) fp16
    (turbo_quantize.py:139-178)."""
    if group_size != 32:
        raise ValueError("the fused kernel's value format has 32-dim groups")
    ext._require_device(values)
    B, H, N, D = values.shape
    dev = values.device
    v = values if values.dtype in (torch.float16, torch.bfloat16, torch.float32) else values.half()
    v = v.contiguous()
    packed = torch.empty((B, H, N, D // 4), dtype=torch.uint8, device=dev)
    scales = torch.empty((B, H, N, D // 32), dtype=torch.float16, device=dev)
    if v.numel() == 0:
        return packed, scales
    lib = _lib.load()
    with torch.cuda.device(dev):
        check(lib.fkv_turbo_compress_values(ptr(v), dtype_code(v.dtype), B * H * N, D, ptr(packed), ptr(scales),
                                            _lib.stream_ptr(dev)), "fkv_turbo_compress_values")
    return packed, scales


# ---------------------------------------------------------------------------
# dequantisation and scores (the reference formulation, torch ops)
# ---------------------------------------------------------------------------

_VAL_LEVELS = (-1.0, -1.0 / 3.0, 1.0 / 3.0, 1.0)  # turbo_quantize.py:16


def _unpack_2bit(packed):
    p = packed.to(torch.int32)
    out = torch.stack([(p >> (2 * i)) & 3 for i in range(4)], dim=-1)
    return out.reshape(packed.shape[:-1] + (packed.shape[-1] * 4,))


def _unpack_1bit(packed):
    p = packed.to(torch.int32)
    out = torch.stack([(p >> i) & 1 for i in range(8)], dim=-1)
    return 2.0 * out.reshape(packed.shape[:-1] + (packed.shape[-1] * 8,)).to(torch.float32) - 1.0


def turbo_dequant_keys(indices_packed, signs_packed, norms, gamma, tc: TurboConstants):
    """norm * (cb[idx] @ Pi) + gamma * (signs @ S) / D -> fp16 (turbo_quantize.py:94-133)."""
    c = tc.on(indices_packed.device)
    idx = _unpack_2bit(indices_packed)
    D = idx.shape[-1]
    k_mse = norms.float().unsqueeze(-1) * (c.centroids[idx] @ c.Pi)
    r_hat = gamma.float().unsqueeze(-1) * (_unpack_1bit(signs_packed) @ c.S) / D
    return (k_mse + r_hat).to(torch.float16)


def turbo_dequant_values(packed, scales, group_size: int = 32):
    """levels[code] * group scale -> fp16 (turbo_quantize.py:181-206)."""
    idx = _unpack_2bit(packed)
    lv = torch.tensor(_VAL_LEVELS, dtype=torch.float32, device=packed.device)[idx]
    sh = lv.shape
    g = lv.reshape(sh[:-1] + (sh[-1] // group_size, group_size))
    return (g * scales.float().unsqueeze(-1)).reshape(sh).to(torch.float16)


def turbo_score_keys(query, indices_packed, signs_packed, norms, gamma, tc: TurboConstants):
    """Logits on compressed keys with GQA groups averaged in the rotated /
    sketched domain (turbo_quantize.py:213-279) -> (B, H_kv, N) fp32."""
    c = tc.on(indices_packed.device)
    q = query.float()
    if q.dim() == 4:
        q = q[:, :, 0, :]
    idx = _unpack_2bit(indices_packed)
    B, Hkv, N, D = idx.shape
    q_rot = q @ c.Pi.T
    q_sk = q @ c.S.T
    if q.shape[1] != Hkv:
        g = q.shape[1] // Hkv
        q_rot = q_rot.reshape(B, Hkv, g, D).mean(2)
        q_sk = q_sk.reshape(B, Hkv, g, D).mean(2)
    mse = norms.float() * (q_rot.unsqueeze(2) * c.centroids[idx]).sum(-1)
    sd = (q_sk.unsqueeze(2) * _unpack_1bit(signs_packed)).sum(-1)
    return mse + (math.sqrt(math.pi / 2) / D) * gamma.float() * sd


# ---------------------------------------------------------------------------
# fused handle (csrc/foveated_attn.cpp:365-491)
# ---------------------------------------------------------------------------


class TurboFoveatedHandle(ext.FoveatedHandle):
    """TurboFoveatedHandle(near_k, near_v, far_k_indices, far_k_signs,
    far_k_norm, far_k_gamma, far_v_packed, far_v_scale, near_valid, Pi,
    S_mat, centroids, spike_margin, metallib_path) (bindings.cpp:103-126):
    copies the tiers into a private device blob; calling it runs the fused
    kernel -> [out (B,Hq,1,D) fp16, spike_flags (B,Hq), spike_tokens (B,Hq)].
    ``metallib_path`` is accepted and ignored."""

    def __init__(self, near_k, near_v, far_k_indices, far_k_signs, far_k_norm, far_k_gamma, far_v_packed,
                 far_v_scale, near_valid, Pi, S_mat, centroids, spike_margin=0.5, metallib_path=""):
        ext._require_device(near_k, near_v, far_k_indices, far_k_signs, far_k_norm, far_k_gamma, far_v_packed,
                            far_v_scale, near_valid)
        if near_k.dim() != 4 or near_k.shape != near_v.shape:
            raise ValueError("near_k/near_v must be (B,H,N,D) with equal shapes")
        B, H, Na, D = near_k.shape
        F = far_k_indices.shape[2]
        want = {"far_k_indices": (B, H, F, D // 4), "far_k_signs": (B, H, F, D // 8), "far_k_norm": (B, H, F),
                "far_k_gamma": (B, H, F), "far_v_packed": (B, H, F, D // 4), "far_v_scale": (B, H, F, D // 32)}
        got = {"far_k_indices": far_k_indices, "far_k_signs": far_k_signs, "far_k_norm": far_k_norm,
               "far_k_gamma": far_k_gamma, "far_v_packed": far_v_packed, "far_v_scale": far_v_scale}
        for name, shp in want.items():
            if tuple(got[name].shape) != shp:
                raise ValueError(f"{name} {tuple(got[name].shape)} does not match near {tuple(near_k.shape)}: want {shp}")
        self.device = near_k.device
        self.B, self.H_kv, self.D, self.N_near, self.N_far = B, H, D, Na, F
        self.spike_margin = float(spike_margin)
        nk = near_k.contiguous()
        nv = near_v.to(nk.dtype).contiguous()
        if nk.dtype not in (torch.float16, torch.bfloat16, torch.float32):
            nk, nv = nk.half(), nv.half()
        nz = far_k_norm.dtype if far_k_norm.dtype in (torch.float16, torch.bfloat16, torch.float32) else torch.float16
        kn = far_k_norm.to(nz).contiguous()
        kg = far_k_gamma.to(nz).contiguous()
        vs = far_v_scale.to(nz).contiguous()
        ki = far_k_indices.to(torch.uint8).contiguous()
        ks = far_k_signs.to(torch.uint8).contiguous()
        vp = far_v_packed.to(torch.uint8).contiguous()
        valid = near_valid.to(torch.int32).contiguous()
        pi = _f32(torch.as_tensor(Pi), self.device)
        sm = _f32(torch.as_tensor(S_mat), self.device)
        cb = _f32(torch.as_tensor(centroids), self.device)
        if tuple(pi.shape) != (D, D) or tuple(sm.shape) != (D, D) or cb.numel() != 4:
            raise ValueError("Pi and S_mat must be (D, D) and centroids (4,)")
        lib = _lib.load()
        h = ctypes.c_void_p()
        with torch.cuda.device(self.device):
            check(lib.fkv_turbo_create(ctypes.byref(h), B, H, D, Na, F, ptr(nk), ptr(nv), dtype_code(nk.dtype),
                                       ptr(ki), ptr(ks), ptr(kn), ptr(kg), ptr(vp), ptr(vs), dtype_code(nz),
                                       ptr(valid), ptr(pi), ptr(sm), ptr(cb), self.spike_margin,
                                       _lib.stream_ptr(self.device)), "fkv_turbo_create")
        self._h = h
        self._lib = lib


def build_turbo_layer(cfg, keys, values, importance=None):
    """The turbo branch of _assign_and_build_layer (mlx_foveated.py:799-944):
    near tier, archive and indices from the fused compress kernel, the far
    rows (fp16) compressed with TurboQuant; the fp8 far fields stay empty."""
    from .tier_cache import FoveatedLayer, tier_index_tensors

    B, H, S, D = keys.shape
    cl = ext.CompressHandle(cfg.to_native()).compress_layer(keys, values, importance=importance)
    if cl.near_idx is not None:
        near_idx, far_idx = cl.near_idx, cl.far_idx
    else:
        near_idx, far_idx = tier_index_tensors(cfg.tier_boundaries(S), S, B, H, keys.device)
    tc = get_turbo_constants(D)
    dev = keys.device
    ki, ks, kn, kg = turbo_compress_keys(cl.archive_k, tc)
    vp, vs = turbo_compress_values(cl.archive_v)
    empty_u8 = torch.zeros((B, H, 0, D), dtype=torch.uint8, device=dev)
    return FoveatedLayer(near_k=cl.near_k, near_v=cl.near_v, near_idx=near_idx, far_k=empty_u8,
                         far_v=torch.zeros((B, H, 0, D // 2), dtype=torch.uint8, device=dev),
                         far_v_scale=torch.zeros((B, H, 0), dtype=torch.float16, device=dev),
                         far_v_zero=torch.zeros((B, H, 0), dtype=torch.float16, device=dev),
                         far_idx=far_idx, archive_k=cl.archive_k, archive_v=cl.archive_v, archive_idx=far_idx,
                         near_valid=cl.near_valid, compress_method="turbo", turbo_far_k_indices=ki,
                         turbo_far_k_signs=ks, turbo_far_k_norm=kn, turbo_far_k_gamma=kg, turbo_far_v_packed=vp,
                         turbo_far_v_scale=vs, _turbo_constants=tc)
