"""ctypes binding of the gfx950 C-ABI library ``libfkv.so`` (include/fkv.h).

The library is built in-tree by ``foveated_kv_amd/csrc/Makefile`` (or
``__graft_entry__.build()``).  There is no fallback: if the library is
missing or does not load, every entry point raises ``FkvLibraryError``.

torch is imported before the library is loaded so that the HIP runtime
torch ships (``libamdhip64.so.7``) is the one the library binds to; device
pointers and streams come from torch tensors / streams.
"""

import ctypes
import os

import torch  # noqa: F401  (binds the process to torch's HIP runtime first)

_HERE = os.path.dirname(os.path.abspath(__file__))
# FKV_LIBRARY selects another build of the library (e.g. the phase-stamp
# build, libfkv_stamps.so, that bench.py --phase-stamps reads)
LIB_PATH = os.environ.get("FKV_LIBRARY") or os.path.join(_HERE, "libfkv.so")

FKV_OK = 0
FKV_EINVAL = -1
FKV_EHIP = -2
FKV_ENOMEM = -3
FKV_EDATA = -4

FKV_F16 = 0
FKV_BF16 = 1
FKV_F32 = 2


class FkvLibraryError(RuntimeError):
    """The HIP library is missing, failed to load, or a call failed."""


class FkvDataError(ValueError):
    """Input data outside what the reference encoder can produce."""


class TierConfigC(ctypes.Structure):
    _fields_ = [
        ("near_pct", ctypes.c_double),
        ("n_sinks", ctypes.c_int32),
        ("window_size", ctypes.c_int32),
        ("promo_headroom_pct", ctypes.c_double),
        ("promo_headroom_min", ctypes.c_int32),
        ("v_group", ctypes.c_int32),
        ("k_scale", ctypes.c_int32),
    ]


class TiersC(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in (
        "n_sinks", "window", "near_from_mid", "far_count", "r_actual", "n_near_padded",
        "mid_start", "mid_end", "near_mid_start", "headroom")]


class BlobInfoC(ctypes.Structure):
    _fields_ = [
        ("blob", ctypes.c_void_p),
        ("blob_bytes", ctypes.c_uint64),
        ("near_k_offset", ctypes.c_uint64),
        ("near_v_offset", ctypes.c_uint64),
        ("near_valid_offset", ctypes.c_uint64),
        ("n_near_alloc", ctypes.c_int32),
        ("n_far", ctypes.c_int32),
        ("B", ctypes.c_int32),
        ("H_kv", ctypes.c_int32),
        ("D", ctypes.c_int32),
    ]


# name -> (restype, argtypes); every symbol include/fkv.h declares
P = ctypes.c_void_p
I32 = ctypes.c_int32
F32 = ctypes.c_float
SIGNATURES = {
    "fkv_is_available": (ctypes.c_int, []),
    "fkv_last_error": (ctypes.c_char_p, []),
    "fkv_version": (ctypes.c_int, []),
    "fkv_tier_boundaries": (ctypes.c_int, [ctypes.POINTER(TierConfigC), I32, ctypes.POINTER(TiersC)]),
    "fkv_compress_layer": (ctypes.c_int, [ctypes.POINTER(TierConfigC), P, P, I32, I32, I32, I32, I32,
                                          P, P, P, P, P, P, P, P, P, P]),
    "fkv_partition_importance": (ctypes.c_int, [ctypes.POINTER(TierConfigC), P, I32, I32, I32, P, P, P]),
    "fkv_compress_layer_indexed": (ctypes.c_int, [ctypes.POINTER(TierConfigC), P, P, I32, I32, I32, I32, I32,
                                                  P, P, P, P, P, P, P, P, P, P, P, P]),
    "fkv_compress_layer_ex": (ctypes.c_int, [ctypes.POINTER(TierConfigC), P, P, I32, I32, I32, I32, I32,
                                             P, P, P, P, P, P, P, P, P, P, P, P, P]),
    "fkv_attn_create": (ctypes.c_int, [ctypes.POINTER(P), I32, I32, I32, I32, I32, P, P, I32, P, P, P, P,
                                       I32, P, F32, P]),
    "fkv_attn_create_g32": (ctypes.c_int, [ctypes.POINTER(P), I32, I32, I32, I32, I32, P, P, I32, P, P, P, P,
                                           I32, P, F32, P]),
    "fkv_turbo_create": (ctypes.c_int, [ctypes.POINTER(P), I32, I32, I32, I32, I32, P, P, I32, P, P, P, P, P,
                                        P, I32, P, P, P, P, F32, P]),
    "fkv_turbo_compress_keys": (ctypes.c_int, [P, I32, ctypes.c_int64, I32, P, P, P, P, P, P, P, P, P]),
    "fkv_turbo_compress_values": (ctypes.c_int, [P, I32, ctypes.c_int64, I32, P, P, P]),
    "fkv_attn_call": (ctypes.c_int, [P, P, I32, I32, P, P, I32, P, P, P, P]),
    "fkv_attn_call_dev": (ctypes.c_int, [P, P, I32, I32, P, P, P, I32, P, P, P, P]),
    "fkv_attn_call_strided": (ctypes.c_int, [P, P, I32, I32, P, P, I32, I32, P, P, P, P]),
    "fkv_attn_call_noalloc": (ctypes.c_int, [P, P, I32, I32, P, P, I32, P, P, P, P]),
    "fkv_attn_plan": (ctypes.c_int, [I32, I32, I32, I32, I32, I32, I32, I32, I32, P]),
    "fkv_far_plan": (ctypes.c_int, [I32, I32, I32, ctypes.c_int64, ctypes.c_int64, I32, P, P, P]),
    "fkv_attn_blob_info": (ctypes.c_int, [P, ctypes.POINTER(BlobInfoC)]),
    "fkv_attn_read_near_valid": (ctypes.c_int, [P, P, P]),
    "fkv_attn_dispatch_info": (ctypes.c_int, [P, ctypes.POINTER(I32)]),
    "fkv_attn_dispatch_check": (ctypes.c_int, [P, ctypes.POINTER(I32), P]),
    "fkv_xcd_rule_fit": (ctypes.c_int, [P, I32, ctypes.POINTER(I32), ctypes.POINTER(I32)]),
    "fkv_phase_stamps": (ctypes.c_int, [P, I32, I32]),
    "fkv_xcd_watch_violations": (ctypes.c_int32, [P, I32]),
    "fkv_attn_destroy": (None, [P]),
    "fkv_attn_set_k_scale": (ctypes.c_int, [P, P, P]),
    "fkv_attn_set_spike_k": (ctypes.c_int, [P, I32]),
    "fkv_e4m3_decode": (ctypes.c_int, [P, P, ctypes.c_int64, P]),
    "fkv_hbm_read_probe": (ctypes.c_int, [P, ctypes.c_int64, I32, I32, I32, P, P]),
    "fkv_attn_promote_rows": (ctypes.c_int, [P, I32, P, P, P, I32, P]),
    "fkv_attn_export_near": (ctypes.c_int, [P, P, P, P]),
    "fkv_promoter_create": (ctypes.c_int, [I32, I32, I32, ctypes.POINTER(P)]),
    "fkv_promoter_set_spike_k": (ctypes.c_int, [P, I32]),
    "fkv_promoter_register_archive": (ctypes.c_int, [P, I32, P, P, I32, I32, I32, I32, P, I32]),
    "fkv_promoter_register_archive_device": (ctypes.c_int, [P, I32, P, P, I32, I32, I32, I32, P]),
    "fkv_promoter_register_archive_files": (ctypes.c_int, [P, I32, ctypes.c_char_p, ctypes.c_char_p, I32, I32,
                                                           I32, P]),
    "fkv_promoter_register_handle": (ctypes.c_int, [P, I32, P, P]),
    "fkv_promoter_drain_device": (ctypes.c_int, [P, I32, P, P, P, I32, I32, I32, I32, I32, P, I32, P]),
    "fkv_promoter_drain": (ctypes.c_int, [P, I32, P, P, P, I32, I32, I32, I32, I32]),
    "fkv_promoter_pending": (ctypes.c_int, [P, P, I32]),
    "fkv_promoter_flush": (ctypes.c_int, [P]),
    "fkv_promoter_order": (ctypes.c_int, [P, I32, P]),
    "fkv_promoter_synchronize": (ctypes.c_int, [P]),
    "fkv_promoter_get_stats": (ctypes.c_int, [P, P]),
    "fkv_promoter_near_valid": (ctypes.c_int, [P, I32, P, I32]),
    "fkv_promoter_destroy": (None, [P]),
}

STATS_FIELDS = ("spikes_detected", "spikes_queued", "spikes_deduplicated", "spikes_cooled_down",
                "promotions_completed", "promotions_headroom_full")


class PromoterStatsC(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint64) for n in STATS_FIELDS]

_lib = None
_load_error = None


def load():
    """Load libfkv.so once; raise FkvLibraryError if it is unavailable."""
    global _lib, _load_error
    if _lib is not None:
        return _lib
    if _load_error is not None:
        raise FkvLibraryError(_load_error)
    if not os.path.exists(LIB_PATH):
        _load_error = (f"{LIB_PATH} is not built; run `make -C foveated_kv_amd/csrc` "
                       "or __graft_entry__.build()")
        raise FkvLibraryError(_load_error)
    try:
        lib = ctypes.CDLL(LIB_PATH)
    except OSError as e:
        _load_error = f"cannot load {LIB_PATH}: {e}"
        raise FkvLibraryError(_load_error) from e
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def check(rc, what=""):
    if rc == FKV_OK:
        return
    msg = load().fkv_last_error().decode(errors="replace")
    if rc == FKV_EDATA:
        raise FkvDataError(f"{what}: {msg}")
    raise FkvLibraryError(f"{what} failed ({rc}): {msg}")


def dtype_code(t):
    if t == torch.float16:
        return FKV_F16
    if t == torch.bfloat16:
        return FKV_BF16
    if t == torch.float32:
        return FKV_F32
    raise TypeError(f"unsupported dtype {t}")


def ptr(t):
    """Device pointer of a tensor (None for empty / None)."""
    if t is None or t.numel() == 0:
        return None
    return ctypes.c_void_p(t.data_ptr())


def stream_ptr(device=None):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)
