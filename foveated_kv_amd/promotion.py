"""Promotion of far-tier tokens into near-tier headroom.

Mirror of the reference's ``foveated_ext.PromotionPipeline``
(samfurr/foveated_kv csrc/bindings.cpp:42-100, csrc/promotion_pipeline.cpp)
on the gfx950 library: the same constructor defaults, method names and
statistics.  ``drain_spikes`` runs the reference's filter on the host (GQA
dedup, cooldown, position dedup, per-call budget); the copy of exact fp16
rows from the host-pinned archive into the blob's near headroom and the
``near_valid[h]`` bump run as stream-ordered device work on a side stream
(``flush``), ordered before the layer's next attention launch by
``order``.
"""

import ctypes

import numpy as np
import torch

from . import _lib
from ._lib import check


def _host_i32(t):
    """int32 host copy of a tensor / array (C-contiguous numpy)."""
    if isinstance(t, torch.Tensor):
        t = t.detach().to("cpu", torch.int32)
        return np.ascontiguousarray(t.numpy())
    return np.ascontiguousarray(np.asarray(t, dtype=np.int32))


def _np_ptr(a):
    return a.ctypes.data_as(ctypes.c_void_p) if a is not None and a.size else None


class PromotionPipeline:
    """PromotionPipeline(n_layers, cooldown_steps=5, max_per_drain=8).

    Differences from the reference kept deliberately small: there is no
    worker thread -- ``drain_spikes`` queues records and (by default)
    ``flush``es them as asynchronous GPU work; call ``order(layer)`` before a
    layer's next attention launch (the fused attention path does) so the
    promoted rows and the new ``near_valid`` are seen together.
    """

    def __init__(self, n_layers, cooldown_steps=5, max_per_drain=8, spike_k=1):
        """``spike_k`` (an extension, see fkv_promoter_set_spike_k): spiking
        tokens per query head the drains take, matching the attention
        handles' spike_k (1: the reference's single token)."""
        self._lib = _lib.load()
        h = ctypes.c_void_p()
        check(self._lib.fkv_promoter_create(int(n_layers), int(cooldown_steps), int(max_per_drain), ctypes.byref(h)),
              "fkv_promoter_create")
        self._h = h
        check(self._lib.fkv_promoter_set_spike_k(h, int(spike_k)), "fkv_promoter_set_spike_k")
        self.spike_k = int(spike_k)
        self.n_layers = int(n_layers)
        self._keep = {}  # layer -> host arrays the C side borrows
        self._device_archives = {}  # layer -> GPU archive rows the C side borrows
        self._handles = {}
        self._stopped = False

    def __del__(self):
        h = getattr(self, "_h", None)
        if h is not None and h.value:
            self._lib.fkv_promoter_destroy(h)
            self._h = None

    # ---- registration ----
    def register_archive(self, layer_idx, path_k, path_v, H_kv, S_arc, D, archive_idx):
        """From the reference's on-disk archive files ((H_kv, S_arc, D) fp16,
        disk_archive.py:127-185).  Like the reference, an unusable archive is
        not an error: the layer is left without one and its drains are no-ops."""
        idx = _host_i32(archive_idx).reshape(-1)
        self._device_archives.pop(int(layer_idx), None)
        rc = self._lib.fkv_promoter_register_archive_files(self._h, int(layer_idx), str(path_k).encode(),
                                                           str(path_v).encode(), int(H_kv), int(S_arc), int(D),
                                                           _np_ptr(idx))
        return rc == _lib.FKV_OK

    def register_archive_tensors(self, layer_idx, archive_k, archive_v, archive_idx, device=False):
        """From archive rows (B, H_kv, S_arc, D) fp16 on any device (e.g. a
        compressed layer's ``archive_k/v``) and ``archive_idx`` (B, H_kv, S_arc)
        or (H_kv, S_arc).  By default the rows are copied into pinned host
        memory, the reference's placement.  device=True keeps them in GPU
        memory (fp16, contiguous; the pipeline holds a reference), so the
        device drain reads promoted rows from HBM instead of over PCIe
        (fkv_promoter_register_archive_device; no counterpart in the
        reference)."""
        if device:
            if not (archive_k.is_cuda and archive_v.is_cuda):
                raise ValueError("register_archive_tensors(device=True): the rows must be GPU tensors")
            k = archive_k.detach().to(torch.float16).contiguous()
            v = archive_v.detach().to(torch.float16).contiguous()
        else:
            k = archive_k.detach().to("cpu", torch.float16).contiguous()
            v = archive_v.detach().to("cpu", torch.float16).contiguous()
        if k.dim() == 3:
            k, v = k[None], v[None]
        B, H, S, D = k.shape
        idx = _host_i32(archive_idx)
        if idx.ndim == 3:
            idx = np.ascontiguousarray(idx[0])
        if device:
            check(self._lib.fkv_promoter_register_archive_device(self._h, int(layer_idx),
                                                                 ctypes.c_void_p(k.data_ptr()),
                                                                 ctypes.c_void_p(v.data_ptr()), B, H, S, D,
                                                                 _np_ptr(idx)),
                  "fkv_promoter_register_archive_device")
            self._device_archives[int(layer_idx)] = (k, v)  # borrowed by the pipeline: kept alive here
        else:
            check(self._lib.fkv_promoter_register_archive(self._h, int(layer_idx), ctypes.c_void_p(k.data_ptr()),
                                                          ctypes.c_void_p(v.data_ptr()), B, H, S, D, _np_ptr(idx),
                                                          1),
                  "fkv_promoter_register_archive")
            self._device_archives.pop(int(layer_idx), None)

    def register_blob(self, layer_idx, info):
        """``info``: a FoveatedHandle or the BlobWriteInfo of one."""
        handle = getattr(info, "handle", info)
        with torch.cuda.device(handle.device):
            check(self._lib.fkv_promoter_register_handle(self._h, int(layer_idx), handle._h,
                                                         _lib.stream_ptr(handle.device)),
                  "fkv_promoter_register_handle")
        self._handles[int(layer_idx)] = handle

    # ---- per step ----
    def drain_spikes(self, layer_idx, spike_flags, spike_tokens, far_idx, current_step, flush=True):
        """promotion_pipeline.cpp:99-175; spike outputs (B, H_q) (tokens (B,
        H_q, spike_k) when spike_k > 1) and far_idx (B, H_kv, N_far).
        Returns the number of promotions queued."""
        if self._stopped:
            return 0
        if isinstance(spike_flags, torch.Tensor) and isinstance(spike_tokens, torch.Tensor) and \
                spike_flags.is_cuda and spike_tokens.is_cuda:
            # one device-to-host copy (one synchronisation) for both outputs
            both = torch.cat([spike_flags.to(torch.int32).reshape(-1),
                              spike_tokens.to(torch.int32).reshape(-1)]).cpu().numpy()
            nf = spike_flags.numel()
            flags = np.ascontiguousarray(both[:nf].reshape(tuple(spike_flags.shape)))
            tokens = np.ascontiguousarray(both[nf:])
        else:
            flags = _host_i32(spike_flags)
            tokens = _host_i32(spike_tokens)
        fidx = _host_i32(far_idx)
        B, Hq = flags.shape[0], flags.shape[1]
        Hkv, n_far = fidx.shape[1], fidx.shape[2]
        if tokens.size != B * Hq * self.spike_k:
            raise ValueError(f"spike_tokens must hold B*Hq*spike_k = {B * Hq * self.spike_k} tokens, got {tokens.size}")
        n = self._lib.fkv_promoter_drain(self._h, int(layer_idx), _np_ptr(flags), _np_ptr(tokens), _np_ptr(fidx),
                                         B, Hq, Hkv, n_far, int(current_step))
        if n < 0:
            check(n, "fkv_promoter_drain")
        if flush:
            self.flush()
        return n

    def drain_spikes_device(self, layer_idx, spike_flags, spike_tokens, far_idx, current_step, advance_step=False):
        """The same drain and promotion as ``drain_spikes`` + ``flush``, as one
        kernel on torch's current stream of the tensors' device: spike outputs
        (B, H_q) and far_idx (B, H_kv, N_far) int32 stay in device memory and
        nothing waits for the host; the layer's next attention launch on that
        stream sees the promoted rows.  Needs the archive registered with
        ``register_archive_tensors`` (pinned copy) or from files.  A layer
        drained here cannot also be drained by ``drain_spikes`` (the library
        rejects the second kind of drain on a layer).  ``advance_step`` (with a
        device step): the stream's work then stores step + 1 into
        ``current_step`` once the drain has read it, so a captured decode
        step needs no separate counter update."""
        if self._stopped:
            return
        for t in (spike_flags, spike_tokens, far_idx):
            if not (isinstance(t, torch.Tensor) and t.is_cuda and t.dtype == torch.int32 and t.is_contiguous()):
                raise TypeError("drain_spikes_device takes contiguous int32 device tensors")
        B, Hq = spike_flags.shape[0], spike_flags.shape[1]
        Hkv, n_far = far_idx.shape[1], far_idx.shape[2]
        if spike_tokens.numel() != B * Hq * self.spike_k:
            raise ValueError(f"spike_tokens must hold B*Hq*spike_k = {B * Hq * self.spike_k} tokens")
        dev = spike_flags.device
        # the step: a host int, or a device int32 tensor (read by the kernel)
        step_dev = current_step if isinstance(current_step, torch.Tensor) else None
        if step_dev is not None and not (step_dev.is_cuda and step_dev.dtype == torch.int32):
            raise TypeError("a device step must be an int32 device tensor")
        if advance_step and step_dev is None:
            raise TypeError("advance_step needs the step as an int32 device tensor")
        with torch.cuda.device(dev):
            check(self._lib.fkv_promoter_drain_device(self._h, int(layer_idx), _lib.ptr(spike_flags),
                                                      _lib.ptr(spike_tokens), _lib.ptr(far_idx), B, Hq, Hkv, n_far,
                                                      0 if step_dev is not None else int(current_step),
                                                      _lib.ptr(step_dev), 1 if advance_step else 0,
                                                      _lib.stream_ptr(dev)),
                  "fkv_promoter_drain_device")
        self._keep[("dev", int(layer_idx))] = (spike_flags, spike_tokens, far_idx)

    def pending(self):
        """Queued, unflushed records: int32 (n, 4) = layer, head, archive row, position."""
        n = self._lib.fkv_promoter_pending(self._h, None, 0)
        out = np.zeros((max(n, 0), 4), np.int32)
        if n > 0:
            self._lib.fkv_promoter_pending(self._h, _np_ptr(out), n)
        return out

    def flush(self):
        check(self._lib.fkv_promoter_flush(self._h), "fkv_promoter_flush")

    def order(self, layer_idx, stream=None):
        """Make ``stream`` (default: torch's current stream) wait for the
        layer's last flushed promotion."""
        s = stream if stream is not None else torch.cuda.current_stream()
        check(self._lib.fkv_promoter_order(self._h, int(layer_idx), ctypes.c_void_p(s.cuda_stream)),
              "fkv_promoter_order")

    def synchronize(self):
        check(self._lib.fkv_promoter_synchronize(self._h), "fkv_promoter_synchronize")

    def near_valid(self, layer_idx):
        buf = (ctypes.c_uint32 * 4096)()
        n = self._lib.fkv_promoter_near_valid(self._h, int(layer_idx), ctypes.cast(buf, ctypes.c_void_p), 4096)
        if n < 0:
            check(n, "fkv_promoter_near_valid")
        return list(buf[:n])

    def get_stats(self):
        c = _lib.PromoterStatsC()
        check(self._lib.fkv_promoter_get_stats(self._h, ctypes.byref(c)), "fkv_promoter_get_stats")
        return {f: int(getattr(c, f)) for f in _lib.STATS_FIELDS}

    def stop(self):
        """bindings.cpp:97-99: no further promotions; in-flight copies complete."""
        self._stopped = True
        if self._h is not None and self._h.value:
            self.synchronize()
