"""CPU oracle for the FoveatedKV decode hot path -- TEST INFRASTRUCTURE ONLY.

This package restates the reference algorithm (samfurr/foveated_kv) on the
CPU.  Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import it, and only as the checker.  The product
package ``foveated_kv_amd`` never imports it and has no CPU fallback.

The heavy arithmetic lives in ``fkv_oracle.c`` (built by ``oracle/Makefile``
into ``oracle/_build/libfkv_oracle.so``); this module wraps it for numpy
arrays.  TurboQuant constants and compression (pure numpy/scipy, as the
reference computes them) are in ``oracle.turbo``.

Parity status per function is listed at the top of ``fkv_oracle.c``; the
tests that pin each one are in ``tests/test_oracle_*.py``.
"""

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "libfkv_oracle.so")
_lib = None


def build():
    """Compile the C restatement with the committed Makefile."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def _load():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(_LIB_PATH):
        build()
    lib = ctypes.CDLL(_LIB_PATH)
    P = ctypes.c_void_p
    I = ctypes.c_int
    I64 = ctypes.c_int64
    lib.orc_fp16_to_e4m3.restype = ctypes.c_uint8
    lib.orc_fp16_to_e4m3.argtypes = [ctypes.c_uint16]
    lib.orc_fp16_to_e4m3_py.restype = ctypes.c_uint8
    lib.orc_fp16_to_e4m3_py.argtypes = [ctypes.c_uint16]
    lib.orc_e4m3_to_fp16.restype = ctypes.c_uint16
    lib.orc_e4m3_to_fp16.argtypes = [ctypes.c_uint8]
    lib.orc_d2h.restype = ctypes.c_uint16
    lib.orc_d2h.argtypes = [ctypes.c_double]
    lib.orc_encode_fp8.restype = None
    lib.orc_encode_fp8.argtypes = [P, P, I64, I]
    lib.orc_quant_int4_rows.restype = None
    lib.orc_quant_int4_rows.argtypes = [P, I64, I, P, P, P]
    lib.orc_quant_int4_rows_py.restype = None
    lib.orc_quant_int4_rows_py.argtypes = [P, I64, I, P, P, P]
    lib.orc_tier_boundaries.restype = None
    lib.orc_tier_boundaries.argtypes = [ctypes.c_double, I, I, ctypes.c_double, I, I, P]
    lib.orc_split_plan.restype = None
    lib.orc_split_plan.argtypes = [I, P]
    lib.orc_attend_kernel.restype = I
    lib.orc_attend_kernel.argtypes = [I] * 7 + [P] * 12 + [ctypes.c_float, I, I, I, I] + [P] * 6
    lib.orc_attend_formulation.restype = I
    lib.orc_attend_formulation.argtypes = [I] * 7 + [P, I] + [P] * 9 + [I, P, P]
    lib.orc_compress_foveal.restype = None
    lib.orc_compress_foveal.argtypes = [P, P] + [I] * 9
    _lib = lib
    return lib


def _ptr(a):
    return a.ctypes.data_as(ctypes.c_void_p) if a is not None and a.size else None


def _u16(x):
    """fp16 (or raw uint16) array -> contiguous uint16 view."""
    x = np.ascontiguousarray(x)
    if x.dtype == np.float16:
        return x.view(np.uint16)
    if x.dtype == np.uint16:
        return x
    raise TypeError(f"expected float16/uint16, got {x.dtype}")


# ---------------------------------------------------------------------------
# fp8 / int4 codecs
# ---------------------------------------------------------------------------

def encode_fp8(x, python_semantics=False):
    """fp16 -> E4M3 codes.  Metal encoder (foveated_compress.metal:39-66) by
    default; ``python_semantics`` selects mlx_foveated.py:528-566."""
    lib = _load()
    src = _u16(x)
    dst = np.empty(src.shape, np.uint8)
    lib.orc_encode_fp8(_ptr(src), _ptr(dst), src.size, int(python_semantics))
    return dst


def decode_fp8(codes):
    """E4M3 codes -> fp16 via the kernel LUT (foveated_attn.metal:237-253)."""
    lib = _load()
    table = np.array([lib.orc_e4m3_to_fp16(i) for i in range(256)], np.uint16)
    return table[np.asarray(codes, np.uint8)].view(np.float16)


# The largest value the reference's Metal encoder represents to 3 mantissa
# bits: it emits exponent 15 only as the saturation code 0x7E (448), so every
# input from 240 up (after rounding) lands there (foveated_compress.metal:
# 39-66).  Per-head scales map a head's largest |key| to 240 (code 0x77).
E4M3_TOP = 240.0


def k_head_scale(keys):
    """Per-head fp8 key scale of the benchmark's "per-head-scaled fp8 E4M3"
    keys (an extension; the reference encodes keys unscaled,
    foveated_compress.metal:39-66): keys (..., N, D) fp16 -> scale (...) fp32
    = amax / 240 over the finite values of each head's N x D keys (fp32
    division), 1 where amax is 0 (or N = 0).  240 is the top of the Metal
    encoder's accurate range (E4M3_TOP): with 448, the E4M3 maximum, every
    key in (240, 448] x scale would saturate to 448."""
    x = np.asarray(keys, np.float16).astype(np.float32)
    x = np.where(np.isfinite(x), np.abs(x), np.float32(0))
    amax = x.reshape(x.shape[:-2] + (-1,)).max(axis=-1, initial=np.float32(0)).astype(np.float32)
    return np.where(amax > 0, amax / np.float32(E4M3_TOP), np.float32(1)).astype(np.float32)


def encode_fp8_scaled(keys, scale):
    """Per-head-scaled E4M3 (extension): keys (..., N, D) fp16, scale (...)
    fp32 -> codes of the Metal encoder applied to fp16(key / scale), the
    quotient an fp32 division rounded to fp16 (nearest even).  scale = 1
    gives encode_fp8(keys); with k_head_scale the head's largest finite
    |key| encodes to 0x77 (240)."""
    x = np.asarray(keys, np.float16).astype(np.float32)
    s = np.asarray(scale, np.float32)[..., None, None]
    with np.errstate(over="ignore", invalid="ignore"):
        y = (x / s).astype(np.float16)
    return encode_fp8(y)


def quant_int4(x, python_semantics=False):
    """Per-token INT4 of (..., D) fp16 -> (packed (..., D/2) u8, scale (...) f16,
    zero (...) f16).  Metal semantics (foveated_compress.metal:153-205) by
    default; ``python_semantics`` selects mlx_foveated.py:569-600."""
    lib = _load()
    src = _u16(x)
    D = src.shape[-1]
    rows = src.size // D if D else 0
    lead = src.shape[:-1]
    packed = np.empty(lead + (D // 2,), np.uint8)
    scale = np.empty(lead, np.uint16)
    zero = np.empty(lead, np.uint16)
    fn = lib.orc_quant_int4_rows_py if python_semantics else lib.orc_quant_int4_rows
    if rows:
        fn(_ptr(src), rows, D, _ptr(packed), _ptr(scale), _ptr(zero))
    return packed, scale.view(np.float16), zero.view(np.float16)


def dequant_int4_fp32(packed, scale, zero):
    """fp32 dequant as the fused kernel does it: fma(nibble, scale, zero)."""
    lo = (packed & 15).astype(np.float32)
    hi = (packed >> 4).astype(np.float32)
    codes = np.stack([lo, hi], axis=-1).reshape(packed.shape[:-1] + (packed.shape[-1] * 2,))
    return codes * scale.astype(np.float32)[..., None] + zero.astype(np.float32)[..., None]


# ---------------------------------------------------------------------------
# tiers and split plan
# ---------------------------------------------------------------------------

_TB_KEYS = ("n_sinks", "window", "near_from_mid", "far_count", "R_actual",
            "N_near_padded", "mid_start", "mid_end", "near_mid_start", "headroom")


def tier_boundaries(S, near_pct=0.10, n_sinks=4, window_size=32,
                    promo_headroom_pct=0.5, promo_headroom_min=8):
    """mlx_foveated.py:128-169."""
    lib = _load()
    out = np.zeros(10, np.int32)
    lib.orc_tier_boundaries(float(near_pct), int(n_sinks), int(window_size),
                            float(promo_headroom_pct), int(promo_headroom_min), int(S), _ptr(out))
    d = {k: int(v) for k, v in zip(_TB_KEYS, out)}
    d["far_src_offset"] = d["mid_start"]
    return d


def split_plan(s_total):
    """foveated_attn.cpp:26-38 -> (split_size, num_splits, max_splits)."""
    lib = _load()
    out = np.zeros(3, np.int32)
    lib.orc_split_plan(int(s_total), _ptr(out))
    return tuple(int(v) for v in out)


def tier_indices(S, B, H, **cfg):
    """near_idx (B,H,Npad) with -1 headroom, far_idx (B,H,F) int32:
    mlx_foveated.py:719-752."""
    tb = tier_boundaries(S, **cfg)
    parts = [np.arange(tb["n_sinks"]),
             np.arange(tb["near_mid_start"], tb["mid_end"]),
             np.arange(S - tb["window"], S)]
    near = np.concatenate(parts).astype(np.int32)
    near = np.concatenate([near, np.full(tb["N_near_padded"] - tb["R_actual"], -1, np.int32)])
    far = np.arange(tb["mid_start"], tb["mid_start"] + tb["far_count"], dtype=np.int32)
    return (np.broadcast_to(near, (B, H, near.size)).copy(),
            np.broadcast_to(far, (B, H, far.size)).copy(), tb)


def partition_importance(importance, S, B, H, **cfg):
    """Importance partition (the published benchmark configs' "near = sinks + window +
    top-importance middle"; the reference partitions by recency,
    mlx_foveated.py:128-169, 719-752): per (b, h), the near_from_mid middle
    tokens of highest importance, ties to the later token, NaN below every
    number, -0 == +0.  -> near_idx (B,H,Npad) (sinks, chosen middle
    ascending, window; -1 headroom), far_idx (B,H,F) (rest of the middle,
    ascending), tb."""
    tb = tier_boundaries(S, **cfg)
    imp = np.broadcast_to(np.asarray(importance, np.float32), (B, H, S))
    m0, m1, k = tb["mid_start"], tb["mid_end"], tb["near_from_mid"]
    mid = np.arange(m0, max(m1, m0))
    near = np.full((B, H, tb["N_near_padded"]), -1, np.int32)
    far = np.zeros((B, H, tb["far_count"]), np.int32)
    win = np.arange(S - tb["window"], S)
    for b in range(B):
        for h in range(H):
            v = imp[b, h, mid].astype(np.float64)
            v = np.where(np.isnan(v), -np.inf, v)
            nan = np.isnan(imp[b, h, mid])
            # sort by (not NaN, value, position) descending: NaN last, ties to the later token
            order = np.lexsort((mid, v, ~nan))[::-1]
            chosen = np.sort(mid[order[:k]])
            rest = np.sort(mid[order[k:]])
            seg = np.concatenate([np.arange(tb["n_sinks"]), chosen, win]).astype(np.int32)
            near[b, h, :seg.size] = seg
            far[b, h] = rest
    return near, far, tb


def compress_foveal(x, tb):
    """Near-tier gather (foveated_compress.metal:76-109): (B,H,S,D) fp16 ->
    (B,H,Npad,D) fp16 with zero headroom."""
    lib = _load()
    src = _u16(x)
    B, H, S, D = src.shape
    npad = tb["N_near_padded"]
    dst = np.empty((B, H, npad, D), np.uint16)
    win_start = S - tb["window"] if tb["window"] > 0 else S
    lib.orc_compress_foveal(_ptr(src), _ptr(dst), B * H, S, D, tb["n_sinks"],
                            tb["near_mid_start"], tb["near_from_mid"], win_start,
                            tb["R_actual"], npad)
    return dst.view(np.float16)


def _gather_rows(x, idx):
    """x (B,H,S,D), idx (B,H,N) -> (B,H,N,D) with zero rows where idx < 0."""
    safe = np.where(idx < 0, 0, idx)
    out = np.take_along_axis(x, safe[..., None].astype(np.int64), axis=2)
    out[idx < 0] = 0
    return out


def compress_layer(keys, values, v_group=0, importance=None, k_scale=False, **cfg):
    """The whole fp8 compress of one layer (foveated_compress.cpp:95-201):
    returns dict with near_k/near_v/far_k/far_v/far_v_scale/far_v_zero/
    far_k_scale/near_valid/near_idx/far_idx/archive_k/archive_v/tb.
    v_group = 32 quantises V per 32-dim group (scales (B,H,F,D/32)) instead
    of per token; ``importance`` selects the near middle by
    partition_importance; ``k_scale`` encodes the far keys per-head scaled
    (k_head_scale / encode_fp8_scaled; far_k_scale (B,H) fp32, else None)."""
    keys = np.ascontiguousarray(keys, np.float16)
    values = np.ascontiguousarray(values, np.float16)
    B, H, S, D = keys.shape
    if importance is None:
        near_idx, far_idx, tb = tier_indices(S, B, H, **cfg)
        F = tb["far_count"]
        far_sl = slice(tb["mid_start"], tb["mid_start"] + F)
        fk_src = keys[:, :, far_sl]
        fv_src = values[:, :, far_sl]
        near_k, near_v = compress_foveal(keys, tb), compress_foveal(values, tb)
    else:
        near_idx, far_idx, tb = partition_importance(importance, S, B, H, **cfg)
        fk_src, fv_src = _gather_rows(keys, far_idx), _gather_rows(values, far_idx)
        near_k, near_v = _gather_rows(keys, near_idx), _gather_rows(values, near_idx)
    far_v, fvs, fvz = quant_int4_groups(fv_src, v_group) if v_group else quant_int4(fv_src)
    ks = k_head_scale(fk_src) if k_scale else None
    return {
        "near_k": near_k,
        "near_v": near_v,
        "far_k": encode_fp8_scaled(fk_src, ks) if k_scale else encode_fp8(fk_src),
        "far_k_scale": ks,
        "far_v": far_v,
        "far_v_scale": fvs,
        "far_v_zero": fvz,
        "near_valid": np.full(H, tb["R_actual"], np.int32),
        "near_idx": near_idx,
        "far_idx": far_idx,
        "archive_k": np.ascontiguousarray(fk_src),
        "archive_v": np.ascontiguousarray(fv_src),
        "tb": tb,
    }


# ---------------------------------------------------------------------------
# attention
# ---------------------------------------------------------------------------

def _dec_arrays(B, Hkv, D, dec_k, dec_v):
    if dec_k is None:
        z = np.zeros((B, Hkv, 0, D), np.uint16)
        return z, z, 0
    return _u16(dec_k), _u16(dec_v), dec_k.shape[2]


def _v_group(far_vs, D):
    """0 for per-token scales (B,Hkv,F), else the group size of (B,Hkv,F,D/g) scales."""
    fs = np.asarray(far_vs)
    return 0 if fs.ndim == 3 else D // fs.shape[-1]


def quant_int4_groups(x, group=32, python_semantics=False):
    """INT4 in groups of ``group`` dims: the per-token quantiser applied to
    every group (the group-32 extension) -> packed (..., D/2), scale and zero
    (..., D/group) fp16."""
    x = np.asarray(x)
    sh = x.shape
    rows = x.reshape(sh[:-1] + (sh[-1] // group, group))
    p, s, z = quant_int4(rows, python_semantics=python_semantics)
    return p.reshape(sh[:-1] + (sh[-1] // 2,)), s, z


def attend_kernel(q, near_k, near_v, near_valid, far_k, far_v, far_vs, far_vz,
                  dec_k=None, dec_v=None, spike_margin=10.0, split_size=0,
                  num_splits=0, gate=True, far_k_f16=None, far_k_scale=None,
                  return_far_scores=False):
    """Fused-kernel semantics (foveated_attn.metal:181-432) in fp64.
    q (B,Hq,D) or (B,Hq,1,D) fp16.  ``far_k_f16`` (B,Hkv,F,D) fp16 replaces
    the LUT decode of ``far_k`` when given; ``far_k_scale`` (B,Hkv) fp32
    multiplies each head's decoded far keys (per-head-scaled fp8).  Returns
    (out f64 (B,Hq,D), flags i32, tokens i32, max_far f64, min_near f64),
    plus every far score (B,Hq,F) f64 with ``return_far_scores``."""
    lib = _load()
    q = _u16(q)
    B, Hq = q.shape[:2]
    D = q.shape[-1]
    q = q.reshape(B, Hq, D)
    nk, nv_ = _u16(near_k), _u16(near_v)
    Hkv, Npad = nk.shape[1], nk.shape[2]
    fv = np.ascontiguousarray(far_v, np.uint8)
    F = fv.shape[2]
    fk = np.ascontiguousarray(far_k, np.uint8) if far_k is not None else None
    fk16 = _u16(far_k_f16) if far_k_f16 is not None else None
    fs, fz = _u16(far_vs), _u16(far_vz)
    dk, dv, ndec = _dec_arrays(B, Hkv, D, dec_k, dec_v)
    valid = np.ascontiguousarray(near_valid, np.uint32)
    vg = _v_group(fs, D)
    out = np.zeros((B, Hq, D), np.float64)
    flags = np.zeros((B, Hq), np.int32)
    tokens = np.zeros((B, Hq), np.int32)
    mf = np.zeros((B, Hq), np.float64)
    mn = np.zeros((B, Hq), np.float64)
    ks = None if far_k_scale is None else np.ascontiguousarray(far_k_scale, np.float32).reshape(B, Hkv)
    fsc = np.zeros((B, Hq, F), np.float64) if return_far_scores else None
    rc = lib.orc_attend_kernel(B, Hq, Hkv, D, Npad, F, ndec, _ptr(q), _ptr(nk), _ptr(nv_),
                               _ptr(valid), _ptr(fk), _ptr(fk16), _ptr(fv), _ptr(fs), _ptr(fz),
                               _ptr(dk), _ptr(dv), _ptr(ks), float(spike_margin), int(split_size),
                               int(num_splits), int(bool(gate)), vg, _ptr(out), _ptr(flags),
                               _ptr(tokens), _ptr(mf), _ptr(mn), _ptr(fsc))
    if rc != 0:
        raise ValueError(f"orc_attend_kernel failed: {rc}")
    if return_far_scores:
        return out, flags, tokens, mf, mn, fsc
    return out, flags, tokens, mf, mn


def spike_topk(far_scores, min_near, spike_margin, spike_k):
    """Top-K spike selection (the benchmark's "up to 32 far tokens per head
    per step", an extension of the reference's single token,
    foveated_attn.metal:323-327, 427-430).  far_scores (B,Hq,F), min_near
    (B,Hq).  A far token spikes when its score exceeds min_near + margin.
    Returns counts (B,Hq) int32 = min(K, spiking tokens) and tokens
    (B,Hq,K) int32: the far tokens in descending score order, ties to the
    smaller index (the order the kernel's strict > over ascending tokens
    gives), entries j < count the spiking ones; entry 0 is the first-index
    argmax whatever its score (as the reference's single token; -1 when
    F = 0), entries past the count -1.  K = 1 gives the reference's flag
    and token."""
    fsc = np.asarray(far_scores, np.float64)
    B, Hq, F = fsc.shape
    thr = np.asarray(min_near, np.float64) + float(spike_margin)
    counts = np.zeros((B, Hq), np.int32)
    tokens = np.full((B, Hq, spike_k), -1, np.int32)
    idx = np.arange(F)
    for b in range(B):
        for h in range(Hq):
            if F == 0:
                continue
            order = np.lexsort((idx, -fsc[b, h]))  # score descending, then index ascending
            n = int(min(spike_k, np.count_nonzero(fsc[b, h] > thr[b, h])))
            counts[b, h] = n
            tokens[b, h, :n] = order[:n]
            tokens[b, h, 0] = order[0]
    return counts, tokens


def attend_formulation(q, near_k, near_v, near_valid, far_k, far_v, far_vs, far_vz,
                       dec_k=None, dec_v=None, q_dtype="float16", far_k_scale=None):
    """Reference formulation MLXFoveatedLayer.attend (mlx_foveated.py:239-278)
    in fp64 softmax.  q (B,Hq,D) fp16 bits (or bf16 bits with q_dtype='bfloat16');
    ``far_k_scale`` (B,Hkv) fp32: far keys are decode(code) * scale in fp32."""
    lib = _load()
    q = np.ascontiguousarray(q)
    qb = q.view(np.uint16) if q.dtype != np.uint16 else q
    B, Hq = qb.shape[:2]
    D = qb.shape[-1]
    qb = qb.reshape(B, Hq, D)
    nk, nv_ = _u16(near_k), _u16(near_v)
    Hkv, Npad = nk.shape[1], nk.shape[2]
    fk = np.ascontiguousarray(far_k, np.uint8)
    fv = np.ascontiguousarray(far_v, np.uint8)
    F = fk.shape[2]
    fs, fz = _u16(far_vs), _u16(far_vz)
    dk, dv, ndec = _dec_arrays(B, Hkv, D, dec_k, dec_v)
    valid = np.ascontiguousarray(near_valid, np.uint32)
    out = np.zeros((B, Hq, D), np.float64)
    ks = None if far_k_scale is None else np.ascontiguousarray(far_k_scale, np.float32).reshape(B, Hkv)
    rc = lib.orc_attend_formulation(B, Hq, Hkv, D, Npad, F, ndec, _ptr(qb),
                                    1 if q_dtype == "bfloat16" else 0, _ptr(nk), _ptr(nv_),
                                    _ptr(valid), _ptr(fk), _ptr(fv), _ptr(fs), _ptr(fz),
                                    _ptr(dk), _ptr(dv), _v_group(fs, D), _ptr(ks), _ptr(out))
    if rc != 0:
        raise ValueError(f"orc_attend_formulation failed: {rc}")
    return out


def cosine(a, b):
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    return float(a @ b / (np.linalg.norm(a) * np.linalg.norm(b) + 1e-30))
