"""Two-tier foveated KV cache: the reference's Python tier-cache API on
PyTorch-ROCm (samfurr/foveated_kv src/foveated_kv/mlx_foveated.py:111-968).

  TierConfig        <- MLXTierConfig        (mlx_foveated.py:111-169)
  FoveatedLayer     <- MLXFoveatedLayer     (mlx_foveated.py:172-525)
  FoveatedKVCache   <- MLXFoveatedKVCache   (mlx_foveated.py:603-968)

The ``MLX*`` names are exported as aliases so code written against the
reference imports unchanged.  Compression and fused attention run through
the gfx950 library (``foveated_kv_amd.ext``); there is no CPU or Python
fallback for them -- a missing library raises.  ``attend`` is the
reference formulation (dequant + concat + SDPA, mlx_foveated.py:239-278)
written with torch ops on the cache's device.
"""

import math
from dataclasses import dataclass, field
from typing import Optional

import torch
import torch.nn.functional as F

from . import ext

# Bound at import: the decode closure (foveated_kv_amd.generate) replaces
# torch.nn.functional.scaled_dot_product_attention while installed, and the
# formulation below must keep calling the real function.
_sdpa = F.scaled_dot_product_attention


# ---------------------------------------------------------------------------
# codecs used by the formulation (reference semantics, device torch ops)
# ---------------------------------------------------------------------------

def e4m3_to_fp16(codes: torch.Tensor) -> torch.Tensor:
    """mlx_foveated.py:76-91: exponent 0 -> signed zero, else re-bias by 8."""
    v = codes.to(torch.int32)
    sign = v >> 7
    exp8 = (v >> 3) & 0xF
    mant = v & 0x7
    exp16 = torch.where(exp8 > 0, exp8 + 8, torch.zeros_like(exp8))
    bits = (sign << 15) | (exp16 << 10) | (mant << 7)
    return bits.to(torch.int16).view(torch.float16)


def dequant_int4_per_token(packed, scale, zero):
    """mlx_foveated.py:94-108, in fp16 arithmetic (two roundings).  Scales
    of shape (B,H,N,D/g) (group-g V) apply to their g-dim groups."""
    lo = (packed & 0x0F).to(torch.float16)
    hi = ((packed >> 4) & 0x0F).to(torch.float16)
    B, H, N, Dh = packed.shape
    inter = torch.stack([lo, hi], dim=-1).reshape(B, H, N, Dh * 2)
    if scale.dim() == 4:
        g = Dh * 2 // scale.shape[-1]
        return inter * scale.to(torch.float16).repeat_interleave(g, dim=-1) + \
            zero.to(torch.float16).repeat_interleave(g, dim=-1)
    return inter * scale.to(torch.float16).unsqueeze(-1) + zero.to(torch.float16).unsqueeze(-1)


@dataclass
class TierConfig:
    """Configuration for the 2-tier foveated cache (mlx_foveated.py:111-169)."""

    near_pct: float = 0.10
    n_sinks: int = 4
    window_size: int = 32
    promo_headroom_pct: float = 0.5
    promo_headroom_min: int = 8
    compress_method: str = "fp8"  # "fp8" (fp8 K + int4 V) or "turbo"
    # fp8 far V: one INT4 scale / zero per token (0, the reference) or per
    # 32-dim group (32, the group-32 packed layout)
    v_group: int = 0
    # fp8 far K: unscaled (False, the reference) or per-head scaled (True:
    # scale = amax / 240 per (batch, head), the "per-head-scaled fp8 E4M3")
    k_scale: bool = False
    # spiking far tokens the fused kernel reports per query head (1: the
    # reference's single token; up to 32: "up to 32 far tokens per head per
    # step")
    spike_k: int = 1

    def __post_init__(self):
        if self.compress_method not in ("fp8", "turbo"):
            raise ValueError(
                f"compress_method must be 'fp8' or 'turbo', got '{self.compress_method}'")
        if self.v_group not in (0, 32):
            raise ValueError(f"v_group must be 0 (per token) or 32, got {self.v_group}")
        if not 1 <= int(self.spike_k) <= 32:
            raise ValueError(f"spike_k must be in [1, 32], got {self.spike_k}")
        if self.compress_method == "turbo" and (self.k_scale or self.spike_k != 1):
            raise ValueError("k_scale and spike_k > 1 apply to the fp8 far tier only")

    def tier_boundaries(self, S: int) -> dict:
        n_sinks = min(self.n_sinks, S)
        window = min(self.window_size, max(S - n_sinks, 0))
        near_reserved = n_sinks + window
        R_total = max(int(S * self.near_pct), near_reserved)
        far_count = S - R_total
        if far_count < 0:
            R_total = S
        mid_start = n_sinks
        mid_end = S - window if window > 0 else S
        mid_len = max(mid_end - mid_start, 0)
        near_from_mid = min(max(R_total - near_reserved, 0), mid_len)
        R_actual = n_sinks + near_from_mid + window
        headroom = max(int(R_actual * self.promo_headroom_pct), self.promo_headroom_min)
        near_mid_start = mid_end - near_from_mid
        return {
            "n_sinks": n_sinks,
            "window": window,
            "near_from_mid": near_from_mid,
            "far_count": near_mid_start - mid_start,
            "R_actual": R_actual,
            "N_near_padded": R_actual + headroom,
            "mid_start": mid_start,
            "mid_end": mid_end,
            "near_mid_start": near_mid_start,
            "far_src_offset": mid_start,
        }

    def to_native(self) -> ext.TierConfig:
        c = ext.TierConfig()
        c.near_pct = self.near_pct
        c.n_sinks = self.n_sinks
        c.window_size = self.window_size
        c.promo_headroom_pct = self.promo_headroom_pct
        c.promo_headroom_min = self.promo_headroom_min
        c.v_group = self.v_group
        c.k_scale = 1 if self.k_scale else 0
        return c


class _DecodeBuffer:
    """Append-only fp16 decode tokens (B,H,n,D) in a preallocated device
    buffer (capacity doubles), so each append is one O(1) copy instead of
    re-concatenating the whole buffer (mlx_foveated.py:404-428)."""

    def __init__(self):
        self.k = None
        self.v = None
        self.n = 0

    def append(self, k, v):
        k = k.to(torch.float16)
        v = v.to(torch.float16)
        t = k.shape[2]
        if self.k is None or self.n + t > self.k.shape[2]:
            cap = max(16, 2 * (self.n + t))
            nk = torch.empty(k.shape[:2] + (cap, k.shape[3]), dtype=torch.float16, device=k.device)
            nv = torch.empty_like(nk)
            if self.n:
                nk[:, :, : self.n] = self.k[:, :, : self.n]
                nv[:, :, : self.n] = self.v[:, :, : self.n]
            self.k, self.v = nk, nv
        self.k[:, :, self.n : self.n + t] = k
        self.v[:, :, self.n : self.n + t] = v
        self.n += t

    def views(self):
        if self.n == 0:
            return None, None
        return self.k[:, :, : self.n], self.v[:, :, : self.n]

    def reserve(self, B, H, D, cap, device):
        """Fixed-capacity mode: a zeroed (B,H,cap,D) buffer written by
        ``write_at`` at device-held positions (the host count ``n`` is not
        advanced; the owner sets it when it reads the rows on the host)."""
        self.k = torch.zeros((B, H, cap, D), dtype=torch.float16, device=device)
        self.v = torch.zeros_like(self.k)
        self.n = 0

    def write_at(self, k, v, idx):
        """Rows idx (int64 device tensor of length t) <- k, v (B,H,t,D); no
        host synchronisation, so the write can be captured in a HIP graph."""
        self.k.index_copy_(2, idx, k.to(torch.float16))
        self.v.index_copy_(2, idx, v.to(torch.float16))


@dataclass
class FoveatedLayer:
    """Single-layer 2-tier store (mlx_foveated.py:172-525)."""

    near_k: torch.Tensor  # (B,H,N_near,D) fp16
    near_v: torch.Tensor
    near_idx: torch.Tensor  # (B,H,N_near) int32, -1 for headroom
    far_k: torch.Tensor  # (B,H,F,D) uint8 E4M3
    far_v: torch.Tensor  # (B,H,F,D//2) uint8 INT4
    far_v_scale: torch.Tensor  # (B,H,F) fp16, or (B,H,F,D/32) with group-32 V
    far_v_zero: torch.Tensor
    far_idx: torch.Tensor  # (B,H,F) int32
    archive_k: torch.Tensor = field(repr=False)
    archive_v: torch.Tensor = field(repr=False)
    archive_idx: torch.Tensor = field(repr=False)
    near_valid: Optional[torch.Tensor] = None  # (H,) int32
    compress_method: str = "fp8"
    turbo_far_k_indices: Optional[torch.Tensor] = None
    turbo_far_k_signs: Optional[torch.Tensor] = None
    turbo_far_k_norm: Optional[torch.Tensor] = None
    turbo_far_k_gamma: Optional[torch.Tensor] = None
    turbo_far_v_packed: Optional[torch.Tensor] = None
    turbo_far_v_scale: Optional[torch.Tensor] = None
    _turbo_constants: Optional[object] = None
    far_k_scale: Optional[torch.Tensor] = None  # (B,H) fp32: per-head-scaled fp8 keys
    spike_k: int = 1  # spiking far tokens per query head the fused kernel reports

    def __post_init__(self):
        max_pos = -1
        for t in (self.near_idx, self.far_idx):
            if t.numel() > 0:
                max_pos = max(max_pos, int(t.max().item()))
        self._next_pos = max_pos + 1
        self._decode = _DecodeBuffer()
        if self.near_valid is None:
            self.near_valid = torch.full((self.near_k.shape[1],), self.near_k.shape[2],
                                         dtype=torch.int32, device=self.near_k.device)
        self._kcache = None

    # ---- sizes ----
    @property
    def total_tokens(self) -> int:
        n_near = int(self.near_valid.max().item()) if self.near_valid is not None else self.near_k.shape[2]
        n_far = self.turbo_far_k_norm.shape[2] if self.compress_method == "turbo" else self.far_k.shape[2]
        return n_near + n_far

    # ---- decode buffer ----
    def add_token(self, new_k, new_v) -> None:
        self._decode.append(new_k, new_v)
        self._next_pos += new_k.shape[2]

    @property
    def decode_k(self):
        return self._decode.views()[0]

    @property
    def decode_v(self):
        return self._decode.views()[1]

    @property
    def effective_near_k(self):
        mv = int(self.near_valid.max().item())
        k = self.near_k[:, :, :mv]
        dk = self.decode_k
        return k if dk is None else torch.cat([k, dk], dim=2)

    @property
    def effective_near_v(self):
        mv = int(self.near_valid.max().item())
        v = self.near_v[:, :, :mv]
        dv = self.decode_v
        return v if dv is None else torch.cat([v, dv], dim=2)

    # ---- reference formulation ----
    def _far_dequant(self):
        if self.compress_method == "turbo":
            from .turbo import turbo_dequant_keys, turbo_dequant_values

            return (turbo_dequant_keys(self.turbo_far_k_indices, self.turbo_far_k_signs,
                                       self.turbo_far_k_norm, self.turbo_far_k_gamma,
                                       self._turbo_constants),
                    turbo_dequant_values(self.turbo_far_v_packed, self.turbo_far_v_scale))
        far_k = e4m3_to_fp16(self.far_k)
        if self.far_k_scale is not None:  # per-head-scaled keys: decode * scale in fp32
            far_k = far_k.float() * self.far_k_scale.float()[:, :, None, None]
        return far_k, dequant_int4_per_token(self.far_v, self.far_v_scale, self.far_v_zero)

    def attend(self, query: torch.Tensor) -> torch.Tensor:
        """Dequant + concat + SDPA (mlx_foveated.py:239-312); returns query
        dtype.  Per-head-scaled keys (not representable in fp16) are
        attended to in fp32."""
        far_k, far_v = self._far_dequant()
        cdt = torch.float32 if far_k.dtype == torch.float32 else query.dtype
        near_k, near_v = self.effective_near_k, self.effective_near_v
        all_k = torch.cat([near_k.to(far_k.dtype), far_k], dim=2)
        all_v = torch.cat([near_v, far_v.to(near_v.dtype)], dim=2)
        if all_k.dtype != cdt:
            all_k = all_k.to(cdt)
        if all_v.dtype != cdt:
            all_v = all_v.to(cdt)
        out_dtype = query.dtype
        query = query.to(cdt)
        hq, hkv = query.shape[1], all_k.shape[1]
        if hq != hkv:
            assert hq % hkv == 0
            all_k = all_k.repeat_interleave(hq // hkv, dim=1)
            all_v = all_v.repeat_interleave(hq // hkv, dim=1)
        scale = 1.0 / math.sqrt(query.shape[-1])
        return _sdpa(query, all_k.contiguous(), all_v.contiguous(), scale=scale).to(out_dtype)

    # ---- fused kernel ----
    def _ensure_kcache(self):
        if self._kcache is not None:
            return
        if self.compress_method == "turbo":
            from .turbo import TurboFoveatedHandle

            tc = self._turbo_constants
            handle = TurboFoveatedHandle(
                self.near_k, self.near_v, self.turbo_far_k_indices, self.turbo_far_k_signs,
                self.turbo_far_k_norm, self.turbo_far_k_gamma, self.turbo_far_v_packed,
                self.turbo_far_v_scale, self.near_valid, tc.Pi, tc.S, tc.centroids,
                spike_margin=10.0)
        else:
            handle = ext.FoveatedHandle(self.near_k, self.near_v, self.far_k, self.far_v,
                                        self.far_v_scale, self.far_v_zero, self.near_valid,
                                        spike_margin=10.0, far_k_scale=self.far_k_scale,
                                        spike_k=self.spike_k)
        self._kcache = {"cpp_handle": handle, "B": self.near_k.shape[0],
                        "H_kv": self.near_k.shape[1], "D": self.near_k.shape[-1]}

    def _dispatch_kernel(self, query):
        self._ensure_kcache()
        return self._kcache["cpp_handle"](query, self.decode_k, self.decode_v)

    def attend_fused(self, query):
        return self._dispatch_kernel(query)[0]

    def attend_fused_with_spikes(self, query, spike_margin: float = 0.5):
        """(out, spike_flags, spike_tokens); like the reference the margin
        argument is ignored -- the handle's margin (10.0) applies."""
        return tuple(self._dispatch_kernel(query))

    # ---- device-count decode (graph-captured steps) ----
    def reserve_decode(self, cap: int) -> None:
        """Give the decode buffer a fixed capacity of ``cap`` rows, written at
        device-held positions by ``add_token_at``."""
        B, H, _, D = self.near_k.shape
        self._decode.reserve(B, H, D, cap, self.near_k.device)

    def add_token_at(self, new_k, new_v, idx) -> None:
        self._decode.write_at(new_k, new_v, idx)

    def attend_fused_dev(self, query, n_decode, out=None):
        """The fused kernel over the whole fixed-capacity decode buffer, of
        which the first ``n_decode`` rows (one-element int32 device tensor)
        are valid; results into ``out`` when given."""
        self._ensure_kcache()
        return tuple(self._kcache["cpp_handle"](query, self._decode.k, self._decode.v, n_decode=n_decode,
                                                out=out))

    # ---- python spike detection (mlx_foveated.py:451-499) ----
    def _query_to_kv_heads(self, query):
        q = query[:, :, 0, :] if query.dim() == 4 else query
        n_q, n_kv = q.shape[1], self.near_k.shape[1]
        if n_q == n_kv:
            return q
        g = n_q // n_kv
        return q.reshape(q.shape[0], n_kv, g, q.shape[-1]).mean(dim=2)

    def detect_spikes(self, query, margin: float = 0.5):
        D = query.shape[-1]
        q = self._query_to_kv_heads(query).float()
        near_scores = (q.unsqueeze(2) * self.effective_near_k.float()).sum(-1) / math.sqrt(D)
        threshold = near_scores.min(dim=-1, keepdim=True).values + margin
        if self.far_k.shape[2] == 0:
            return None
        far_scores = (q.unsqueeze(2) * e4m3_to_fp16(self.far_k).float()).sum(-1) / math.sqrt(D)
        mask = far_scores > threshold
        if not bool(mask.any()):
            return None
        res = []
        for b in range(mask.shape[0]):
            for h in range(mask.shape[1]):
                if bool(mask[b, h].any()):
                    res.append([b, h, int(far_scores[b, h].argmax().item())])
        return torch.tensor(res, dtype=torch.int32) if res else None

    def memory_bytes(self) -> dict:
        def nb(t):
            return t.numel() * t.element_size() if t is not None else 0

        near = nb(self.near_k) + nb(self.near_v)
        if self.compress_method == "turbo":
            far = sum(nb(t) for t in (self.turbo_far_k_indices, self.turbo_far_k_signs,
                                      self.turbo_far_k_norm, self.turbo_far_k_gamma,
                                      self.turbo_far_v_packed, self.turbo_far_v_scale))
        else:
            far = nb(self.far_k) + nb(self.far_v) + nb(self.far_v_scale) + nb(self.far_v_zero)
        archive = nb(self.archive_k) + nb(self.archive_v)
        return {"near": near, "far": far, "archive": archive, "total_quantized": near + far,
                "total_with_archive": near + far + archive}


def tier_index_tensors(tb: dict, S: int, B: int, H: int, device):
    """near_idx (B,H,Npad) with -1 headroom and far_idx (B,H,F), int32
    (mlx_foveated.py:719-752)."""
    parts = []
    if tb["n_sinks"] > 0:
        parts.append(torch.arange(tb["n_sinks"], device=device))
    if tb["near_from_mid"] > 0:
        parts.append(torch.arange(tb["near_mid_start"], tb["mid_end"], device=device))
    if tb["window"] > 0:
        parts.append(torch.arange(S - tb["window"], S, device=device))
    near = torch.cat(parts) if parts else torch.zeros(0, dtype=torch.int64, device=device)
    pad = torch.full((tb["N_near_padded"] - tb["R_actual"],), -1, dtype=torch.int64, device=device)
    near = torch.cat([near, pad]).to(torch.int32)
    far = torch.arange(tb["mid_start"], tb["mid_start"] + tb["far_count"], device=device).to(torch.int32)
    return (near.view(1, 1, -1).expand(B, H, -1).contiguous(),
            far.view(1, 1, -1).expand(B, H, -1).contiguous())


class FoveatedKVCache:
    """Multi-layer 2-tier cache (mlx_foveated.py:603-968).

        cache = FoveatedKVCache(cfg)
        cache.update(keys, values, layer_idx)
        stats = cache.compress()
        out = cache.attend_fused(layer_idx, query)
    """

    def __init__(self, cfg: Optional[TierConfig] = None):
        self.cfg = cfg or TierConfig()
        self.layers: list = []
        self._prefill_keys: list = []
        self._prefill_values: list = []
        self._compressed = False
        self.seq_length = 0

    def update(self, key_states, value_states, layer_idx: int):
        while len(self._prefill_keys) <= layer_idx:
            self._prefill_keys.append(None)
            self._prefill_values.append(None)
            self.layers.append(None)
        if self._prefill_keys[layer_idx] is None:
            self._prefill_keys[layer_idx] = key_states
            self._prefill_values[layer_idx] = value_states
        else:
            self._prefill_keys[layer_idx] = torch.cat([self._prefill_keys[layer_idx], key_states], dim=2)
            self._prefill_values[layer_idx] = torch.cat([self._prefill_values[layer_idx], value_states], dim=2)

    def compress(self, query=None, importance=None) -> dict:
        """``importance`` (extension; the reference partitions by recency):
        None, one fp32 tensor broadcastable to (B,H,S) for every layer, or a
        list with one per layer.  The near middle of each (batch, head) is
        then its near_from_mid tokens of highest importance."""
        if not self._prefill_keys:
            return {"compressed": False}
        total_before = total_after = 0
        seq_length = 0
        handle = ext.CompressHandle(self.cfg.to_native()) if self.cfg.compress_method == "fp8" else None
        for i, (keys, values) in enumerate(zip(self._prefill_keys, self._prefill_values)):
            if keys is None:
                continue
            B, H, S, D = keys.shape
            seq_length = S
            total_before += keys.numel() * keys.element_size() * 2
            imp = importance[i] if isinstance(importance, (list, tuple)) else importance
            if self.cfg.compress_method == "turbo":
                from .turbo import build_turbo_layer

                layer = build_turbo_layer(self.cfg, keys, values, importance=imp)
            else:
                layer = self._build_fp8_layer(handle, keys, values, importance=imp)
            self.layers[i] = layer
            total_after += layer.memory_bytes()["total_quantized"]
        self.seq_length = seq_length
        self._prefill_keys.clear()
        self._prefill_values.clear()
        self._compressed = True
        return {"compressed": True, "n_layers": len(self.layers),
                "before_mb": total_before / (1024 * 1024), "after_mb": total_after / (1024 * 1024),
                "compression": total_before / max(total_after, 1)}

    def _build_fp8_layer(self, handle, keys, values, importance=None):
        """_compress_cpp (mlx_foveated.py:679-797) with the fused HIP kernel."""
        B, H, S, D = keys.shape
        cl = handle.compress_layer(keys, values, importance=importance)
        if cl.near_idx is not None:
            near_idx, far_idx = cl.near_idx, cl.far_idx
        else:
            near_idx, far_idx = tier_index_tensors(self.cfg.tier_boundaries(S), S, B, H, keys.device)
        return FoveatedLayer(near_k=cl.near_k, near_v=cl.near_v, near_idx=near_idx, far_k=cl.far_k,
                             far_v=cl.far_v, far_v_scale=cl.far_v_scale, far_v_zero=cl.far_v_zero,
                             far_idx=far_idx, archive_k=cl.archive_k, archive_v=cl.archive_v,
                             archive_idx=far_idx, near_valid=cl.near_valid, far_k_scale=cl.far_k_scale,
                             spike_k=int(self.cfg.spike_k))

    def attend(self, layer_idx: int, query):
        layer = self.layers[layer_idx]
        if layer is None:
            raise ValueError(f"Layer {layer_idx} not initialized")
        return layer.attend(query)

    def attend_fused(self, layer_idx: int, query):
        layer = self.layers[layer_idx]
        if layer is None:
            raise ValueError(f"Layer {layer_idx} not initialized")
        return layer.attend_fused(query)

    def memory_bytes(self) -> dict:
        totals = {"near": 0, "far": 0, "archive": 0}
        for layer in self.layers:
            if layer is None:
                continue
            m = layer.memory_bytes()
            for k in totals:
                totals[k] += m[k]
        totals["total_quantized"] = totals["near"] + totals["far"]
        totals["total_with_archive"] = totals["total_quantized"] + totals["archive"]
        return totals


def standard_attention(query, keys, values):
    """Exact fp16 attention baseline (mlx_foveated.py:971-983)."""
    nq, nkv = query.shape[1], keys.shape[1]
    if nq != nkv:
        keys = keys.repeat_interleave(nq // nkv, dim=1)
        values = values.repeat_interleave(nq // nkv, dim=1)
    return _sdpa(query, keys.contiguous(), values.contiguous(),
                                          scale=1.0 / math.sqrt(query.shape[-1]))


# reference names
MLXTierConfig = TierConfig
MLXFoveatedLayer = FoveatedLayer
MLXFoveatedKVCache = FoveatedKVCache
standard_attention_mlx = standard_attention
