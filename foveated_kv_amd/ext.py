"""Python mirror of the reference's native module ``foveated_ext``
(samfurr/foveated_kv csrc/bindings.cpp:13-159), backed by the gfx950 C-ABI
library instead of nanobind + Metal.

Same class names, argument names, defaults and return shapes:
  TierConfig, CompressedLayer, CompressHandle(cfg).compress_layer/compress_all,
  FoveatedHandle(near_k, ..., near_valid, spike_margin=0.5)(query, dk, dv)
  -> [out, spike_flags, spike_tokens], get_blob_info(), is_available().
Tensors are torch tensors on a ROCm device instead of mx.array.  Every call
is enqueued on torch's current stream of the tensors' device.
"""

import ctypes

import torch

from . import _lib
from ._lib import check, dtype_code, ptr


def is_available():
    """bindings.cpp:158-159 -- True when the library loads and a gfx950 GPU is visible."""
    try:
        lib = _lib.load()
    except _lib.FkvLibraryError:
        return False
    return bool(lib.fkv_is_available())


class TierConfig:
    """C++ TierConfig mirror (csrc/foveated_compress.h:92-98); note the C++
    default promo_headroom_min = 4 (the Python MLXTierConfig default is 8)."""

    def __init__(self):
        self.near_pct = 0.10
        self.n_sinks = 4
        self.window_size = 32
        self.promo_headroom_pct = 0.5
        self.promo_headroom_min = 4
        # far V INT4 scale / zero per token (0, the reference) or per 32-dim
        # group (32): the benchmark's group-32 packed layout
        self.v_group = 0
        # far K E4M3 unscaled (0, the reference) or per-head scaled (1): the
        # benchmark's "per-head-scaled fp8 E4M3" keys, scale = amax / 240
        self.k_scale = 0

    def to_c(self):
        return _lib.TierConfigC(float(self.near_pct), int(self.n_sinks), int(self.window_size),
                                float(self.promo_headroom_pct), int(self.promo_headroom_min),
                                int(self.v_group), int(self.k_scale))


def tier_boundaries_c(cfg, S):
    """fkv_tier_boundaries through the C ABI -> dict with the keys of
    MLXTierConfig.tier_boundaries plus 'headroom'."""
    lib = _lib.load()
    out = _lib.TiersC()
    c = cfg.to_c()
    check(lib.fkv_tier_boundaries(ctypes.byref(c), int(S), ctypes.byref(out)), "fkv_tier_boundaries")
    return {
        "n_sinks": out.n_sinks, "window": out.window, "near_from_mid": out.near_from_mid,
        "far_count": out.far_count, "R_actual": out.r_actual, "N_near_padded": out.n_near_padded,
        "mid_start": out.mid_start, "mid_end": out.mid_end, "near_mid_start": out.near_mid_start,
        "far_src_offset": out.mid_start, "headroom": out.headroom,
    }


def _require_device(*ts):
    for t in ts:
        if t is not None and not t.is_cuda:
            raise TypeError("foveated_kv_amd tensors must live on a ROCm device (got a CPU tensor)")


def _row_stride(k, v):
    """Row capacity of fp16 decode views (B,H,n,D) that are the first n rows
    of (B,H,cap,D) buffers (a growing decode buffer's views), else 0."""
    if k.dtype != torch.float16 or v.dtype != torch.float16 or k.stride() != v.stride():
        return 0
    B, H, n, D = k.shape
    sb, sh, sr, sd = k.stride()
    if sd != 1 or sr != D or sh % D != 0:
        return 0
    cap = sh // D
    if cap < n or (B > 1 and sb != H * sh) or (k.data_ptr() % 16) or (v.data_ptr() % 16):
        return 0
    return cap


class CompressedLayer:
    """csrc/foveated_compress.h:100-118 (+ the fp16 far-row archive)."""

    def __init__(self, near_k, near_v, far_k, far_v, far_v_scale, far_v_zero, near_valid,
                 n_near_actual, archive_k=None, archive_v=None, near_idx=None, far_idx=None,
                 far_k_scale=None):
        self.near_k = near_k
        self.near_v = near_v
        self.far_k = far_k
        self.far_v = far_v
        self.far_v_scale = far_v_scale
        self.far_v_zero = far_v_zero
        self.near_valid = near_valid
        self.n_near_actual = n_near_actual
        self.archive_k = archive_k
        self.archive_v = archive_v
        # (B,H,Npad) / (B,H,F) int32 token positions of an importance
        # partition (None: the recency partition of the tier boundaries)
        self.near_idx = near_idx
        self.far_idx = far_idx
        # (B,H) fp32 per-head key scales of per-head-scaled far keys (None:
        # unscaled keys, the reference)
        self.far_k_scale = far_k_scale


class CompressHandle:
    """CompressHandle (csrc/foveated_compress.cpp:95-227): one fused HIP kernel
    per layer builds near / far / archive tensors.  ``metallib_path`` is
    accepted for signature compatibility and ignored."""

    def __init__(self, cfg=None, metallib_path=""):
        self.cfg = cfg if cfg is not None else TierConfig()

    def compress_layer(self, keys, values, with_archive=True, importance=None):
        """``importance`` (optional, fp32, broadcastable to (B,H,S)): the near
        middle becomes the near_from_mid tokens of highest importance per
        (batch, head), ties to the later token (importance = position gives
        the reference's recency partition); the index sets are returned as
        ``near_idx`` / ``far_idx``."""
        _require_device(keys, values, importance)
        if keys.shape != values.shape or keys.dim() != 4:
            raise ValueError(f"keys/values must be (B,H,S,D) with equal shapes, got {tuple(keys.shape)} / {tuple(values.shape)}")
        B, H, S, D = keys.shape
        tb = tier_boundaries_c(self.cfg, S)
        dev = keys.device
        k = keys.contiguous()
        v = values.contiguous()
        if v.dtype != k.dtype:
            v = v.to(k.dtype)
        if k.dtype not in (torch.float16, torch.bfloat16, torch.float32):
            k = k.to(torch.float16)
            v = v.to(torch.float16)
        F = tb["far_count"]
        npad = tb["N_near_padded"]
        near_k = torch.empty((B, H, npad, D), dtype=torch.float16, device=dev)
        near_v = torch.empty_like(near_k)
        far_k = torch.empty((B, H, F, D), dtype=torch.uint8, device=dev)
        far_v = torch.empty((B, H, F, D // 2), dtype=torch.uint8, device=dev)
        vg = int(self.cfg.v_group)
        fvs = torch.empty((B, H, F, D // vg) if vg else (B, H, F), dtype=torch.float16, device=dev)
        fvz = torch.empty_like(fvs)
        near_valid = torch.empty((H,), dtype=torch.int32, device=dev)
        arc_k = torch.empty((B, H, F, D), dtype=torch.float16, device=dev) if with_archive else None
        arc_v = torch.empty_like(arc_k) if with_archive else None
        ks = torch.empty((B, H), dtype=torch.float32, device=dev) if int(self.cfg.k_scale) else None
        lib = _lib.load()
        c = self.cfg.to_c()
        near_idx = far_idx = None
        with torch.cuda.device(dev):
            if importance is not None:
                near_idx, far_idx = partition_importance(self.cfg, importance, B, H, S)
            check(lib.fkv_compress_layer_ex(
                ctypes.byref(c), ptr(k), ptr(v), dtype_code(k.dtype), B, H, S, D, ptr(near_idx), ptr(far_idx),
                ptr(near_k), ptr(near_v), ptr(far_k), ptr(far_v), ptr(fvs), ptr(fvz), ptr(ks), ptr(near_valid),
                ptr(arc_k), ptr(arc_v), _lib.stream_ptr(dev)), "fkv_compress_layer_ex")
        return CompressedLayer(near_k, near_v, far_k, far_v, fvs, fvz, near_valid, tb["R_actual"],
                               arc_k, arc_v, near_idx, far_idx, far_k_scale=ks)

    def compress_all(self, all_keys, all_values, with_archive=True):
        return [self.compress_layer(k, v, with_archive) for k, v in zip(all_keys, all_values)]


def partition_importance(cfg, importance, B, H, S):
    """fkv_partition_importance: importance (fp32, broadcastable to (B,H,S),
    on the device) -> near_idx (B,H,Npad) int32 (sinks, chosen middle,
    window in ascending position; -1 headroom) and far_idx (B,H,F) int32
    (the rest of the middle, ascending)."""
    _require_device(importance)
    tb = tier_boundaries_c(cfg, S)
    dev = importance.device
    imp = importance.to(torch.float32).expand(B, H, S).contiguous()
    near_idx = torch.empty((B, H, tb["N_near_padded"]), dtype=torch.int32, device=dev)
    far_idx = torch.empty((B, H, tb["far_count"]), dtype=torch.int32, device=dev)
    c = cfg.to_c()
    with torch.cuda.device(dev):
        check(_lib.load().fkv_partition_importance(ctypes.byref(c), ptr(imp), B, H, S, ptr(near_idx),
                                                   ptr(far_idx), _lib.stream_ptr(dev)),
              "fkv_partition_importance")
    return near_idx, far_idx


class BlobWriteInfo:
    """csrc/promotion_pipeline.h:66-73 analogue: where promotions land in the
    device blob (offsets in bytes from ``blob_ptr``)."""

    def __init__(self, c):
        self.blob_ptr = c.blob
        self.blob_bytes = c.blob_bytes
        self.near_k_offset = c.near_k_offset
        self.near_v_offset = c.near_v_offset
        self.near_valid_offset = c.near_valid_offset
        self.N_near_alloc = c.n_near_alloc
        self.N_far = c.n_far
        self.B = c.B
        self.H_kv = c.H_kv
        self.D = c.D


class FoveatedHandle:
    """FoveatedHandle (csrc/foveated_attn.cpp:135-254): copies the static tier
    arrays into a private device blob; calling it launches the fused kernel.
    ``metallib_path`` is accepted for signature compatibility and ignored."""

    spike_k = 1  # spiking far tokens per query head the calls report

    def __init__(self, near_k, near_v, far_k, far_v, far_v_scale, far_v_zero, near_valid,
                 spike_margin=0.5, metallib_path="", far_k_scale=None, spike_k=1):
        """Extensions beyond the reference's arguments (bindings.cpp:20-31):
        ``far_k_scale`` (B,H) fp32, the per-head scales of per-head-scaled
        fp8 keys (CompressedLayer.far_k_scale); ``spike_k`` in [1, 32], the
        spiking far tokens a call reports per query head (1: the
        reference's single token; K > 1: spike_flags hold the counts and
        spike_tokens are (B,Hq,K), see fkv_attn_set_spike_k)."""
        _require_device(near_k, near_v, far_k, far_v, far_v_scale, far_v_zero, near_valid, far_k_scale)
        if near_k.dim() != 4 or near_k.shape != near_v.shape:
            raise ValueError("near_k/near_v must be (B,H,N,D) with equal shapes")
        B, H, Na, D = near_k.shape
        F = far_k.shape[2]
        if tuple(far_k.shape) != (B, H, F, D) or tuple(far_v.shape) != (B, H, F, D // 2):
            raise ValueError(f"far_k {tuple(far_k.shape)} / far_v {tuple(far_v.shape)} do not match near {tuple(near_k.shape)}")
        # per-token V scales (B,H,F) as the reference, or one per 32-dim
        # group (B,H,F,D/32): the group-32 packed layout
        grouped = far_v_scale.dim() == 4
        want = (B, H, F, D // 32) if grouped else (B, H, F)
        if tuple(far_v_scale.shape) != want or tuple(far_v_zero.shape) != want:
            raise ValueError(f"far_v_scale / far_v_zero must be (B,H,F) or (B,H,F,D/32), got "
                             f"{tuple(far_v_scale.shape)} / {tuple(far_v_zero.shape)}")
        self.v_group = 32 if grouped else 0
        self.device = near_k.device
        self.B, self.H_kv, self.D, self.N_near, self.N_far = B, H, D, Na, F
        self.spike_margin = float(spike_margin)
        nk = near_k.contiguous()
        nv = near_v.to(nk.dtype).contiguous()
        if nk.dtype not in (torch.float16, torch.bfloat16, torch.float32):
            nk, nv = nk.half(), nv.half()
        fvs = far_v_scale.contiguous()
        fvz = far_v_zero.to(fvs.dtype).contiguous()
        if fvs.dtype not in (torch.float16, torch.bfloat16, torch.float32):
            fvs, fvz = fvs.half(), fvz.half()
        valid = near_valid.to(torch.int32).contiguous()
        fk = far_k.to(torch.uint8).contiguous()
        fv = far_v.to(torch.uint8).contiguous()
        lib = _lib.load()
        h = ctypes.c_void_p()
        with torch.cuda.device(self.device):
            create = lib.fkv_attn_create_g32 if grouped else lib.fkv_attn_create
            check(create(ctypes.byref(h), B, H, D, Na, F, ptr(nk), ptr(nv), dtype_code(nk.dtype),
                         ptr(fk), ptr(fv), ptr(fvs), ptr(fvz), dtype_code(fvs.dtype), ptr(valid),
                         self.spike_margin, _lib.stream_ptr(self.device)),
                  "fkv_attn_create_g32" if grouped else "fkv_attn_create")
        self._h = h
        self._lib = lib
        self.spike_k = 1
        if far_k_scale is not None:
            if tuple(far_k_scale.shape) != (B, H):
                raise ValueError(f"far_k_scale must be (B,H) = {(B, H)}, got {tuple(far_k_scale.shape)}")
            ks = far_k_scale.to(torch.float32).contiguous()
            with torch.cuda.device(self.device):
                check(lib.fkv_attn_set_k_scale(h, ptr(ks), _lib.stream_ptr(self.device)), "fkv_attn_set_k_scale")
        self.set_spike_k(spike_k)

    def set_spike_k(self, spike_k):
        """Spiking far tokens per query head reported by later calls."""
        check(self._lib.fkv_attn_set_spike_k(self._h, int(spike_k)), "fkv_attn_set_spike_k")
        self.spike_k = int(spike_k)

    def __del__(self):
        h = getattr(self, "_h", None)
        if h is not None and h.value:
            self._lib.fkv_attn_destroy(h)
            self._h = None

    def __call__(self, query, decode_k=None, decode_v=None, n_decode=None, out=None):
        """-> [out (B,Hq,1,D) fp16, spike_flags (B,Hq) int32, spike_tokens (B,Hq) int32]
        (spike_k > 1: spike_flags are spike counts, spike_tokens (B,Hq,K))

        n_decode (optional): a one-element int32 device tensor holding how many
        rows of decode_k/decode_v (then a fixed-capacity buffer) are valid.
        The kernel reads it on the device, so a decode step can be captured
        in a HIP graph once and replayed while the buffer fills.
        out (optional): the three result tensors to write, preallocated with
        the shapes and dtypes above (contiguous); the call then allocates
        nothing for its results and returns them."""
        _require_device(query, decode_k, decode_v, n_decode)
        if query.dim() == 4:
            if query.shape[2] != 1:
                raise ValueError("decode attention takes one query position (B,Hq,1,D)")
            q = query[:, :, 0, :]
        else:
            q = query
        B, Hq, D = q.shape
        if B != self.B or D != self.D:
            raise ValueError(f"query {tuple(query.shape)} does not match the handle (B={self.B}, D={self.D})")
        if q.dtype not in (torch.float16, torch.bfloat16, torch.float32):
            q = q.half()
        q = q.contiguous()
        n_dec = 0
        row_stride = 0
        dk = dv = None
        if decode_k is not None and decode_k.shape[2] > 0:
            n_dec = decode_k.shape[2]
            if tuple(decode_k.shape) != (B, self.H_kv, n_dec, D) or decode_v.shape != decode_k.shape:
                raise ValueError("decode_k/decode_v must be (B,H_kv,n,D)")
            row_stride = _row_stride(decode_k, decode_v) if n_decode is None else 0
            if row_stride:
                dk, dv = decode_k, decode_v  # rows of a larger buffer, attended to in place
            else:
                dk = decode_k.to(torch.float16).contiguous()
                dv = decode_v.to(torch.float16).contiguous()
        if n_decode is not None:
            if n_decode.dtype != torch.int32 or n_decode.numel() != 1:
                raise TypeError("n_decode must be a one-element int32 device tensor")
            if dk is None:
                raise ValueError("a device n_decode needs a decode buffer of nonzero capacity")
        tshape = (B, Hq) if self.spike_k == 1 else (B, Hq, self.spike_k)
        if out is None:
            out = torch.empty((B, Hq, 1, D), dtype=torch.float16, device=self.device)
            flags = torch.empty((B, Hq), dtype=torch.int32, device=self.device)
            tokens = torch.empty(tshape, dtype=torch.int32, device=self.device)
        else:
            out, flags, tokens = out
            for t, shape, dt in ((out, (B, Hq, 1, D), torch.float16), (flags, (B, Hq), torch.int32),
                                 (tokens, tshape, torch.int32)):
                if tuple(t.shape) != shape or t.dtype != dt or not t.is_contiguous() or t.device != self.device:
                    raise ValueError(f"out tensors must be contiguous {shape} {dt} on {self.device}")
        with torch.cuda.device(self.device):
            if row_stride:
                check(self._lib.fkv_attn_call_strided(self._h, ptr(q), dtype_code(q.dtype), Hq, ptr(dk), ptr(dv),
                                                      n_dec, row_stride, ptr(out), ptr(flags), ptr(tokens),
                                                      _lib.stream_ptr(self.device)), "fkv_attn_call_strided")
            elif n_decode is None:
                check(self._lib.fkv_attn_call(self._h, ptr(q), dtype_code(q.dtype), Hq, ptr(dk), ptr(dv), n_dec,
                                              ptr(out), ptr(flags), ptr(tokens), _lib.stream_ptr(self.device)),
                      "fkv_attn_call")
            else:
                check(self._lib.fkv_attn_call_dev(self._h, ptr(q), dtype_code(q.dtype), Hq, ptr(dk), ptr(dv),
                                                  ptr(n_decode), n_dec, ptr(out), ptr(flags), ptr(tokens),
                                                  _lib.stream_ptr(self.device)),
                      "fkv_attn_call_dev")
        return [out, flags, tokens]

    def get_blob_info(self):
        c = _lib.BlobInfoC()
        check(self._lib.fkv_attn_blob_info(self._h, ctypes.byref(c)), "fkv_attn_blob_info")
        info = BlobWriteInfo(c)
        info.handle = self  # register_blob targets this handle
        return info

    def export_near(self):
        """The near tier the kernel attends to (promotions included), row-major
        (B, H_kv, N_near_alloc, D) fp16 K and V."""
        shape = (self.B, self.H_kv, self.N_near, self.D)
        k = torch.empty(shape, dtype=torch.float16, device=self.device)
        v = torch.empty_like(k)
        with torch.cuda.device(self.device):
            check(self._lib.fkv_attn_export_near(self._h, ptr(k), ptr(v), _lib.stream_ptr(self.device)),
                  "fkv_attn_export_near")
        return k, v

    def dispatch_info(self):
        """XCD count of the workgroup -> XCD dispatch rule this handle's split
        merge uses (0: the merge goes through memory)."""
        mod = _lib.I32(0)
        check(self._lib.fkv_attn_dispatch_info(self._h, ctypes.byref(mod)), "fkv_attn_dispatch_info")
        return mod.value

    def dispatch_check(self):
        """Violations of the XCD dispatch rule since the last check (0: every
        XCD-local merge ran within one XCD); any violation switches the
        handle to the merge through memory.  Synchronises the current stream."""
        v = _lib.I32(0)
        with torch.cuda.device(self.device):
            check(self._lib.fkv_attn_dispatch_check(self._h, ctypes.byref(v), _lib.stream_ptr(self.device)),
                  "fkv_attn_dispatch_check")
        return v.value

    def read_near_valid(self):
        """Current per-KV-head near_valid of the blob (host list)."""
        buf = (ctypes.c_uint32 * self.H_kv)()
        with torch.cuda.device(self.device):
            check(self._lib.fkv_attn_read_near_valid(self._h, ctypes.cast(buf, ctypes.c_void_p),
                                                     _lib.stream_ptr(self.device)), "fkv_attn_read_near_valid")
        return list(buf)
