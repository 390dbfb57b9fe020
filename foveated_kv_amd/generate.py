"""Decode-time routing of a PyTorch model's attention through the fused
gfx950 kernel, and the prefill -> compress -> decode loop around it
(samfurr/foveated_kv src/foveated_kv/mlx_generate.py:38-416; its
perplexity and passkey evaluations, :419-590, are model-level and not
rebuilt).

``install_fused_sdpa`` replaces ``torch.nn.functional.scaled_dot_product_attention``
with a closure (mlx_generate.py:84-131):

* a call whose query holds more than one position (prefill) goes to the
  original function unchanged;
* a one-position call (decode) is answered by the next layer's foveated
  handle: a layer counter walks ``fov_cache.layers`` in call order, wraps
  modulo the layer count, and is reset once per step by ``drain_spikes`` /
  ``reset_fused_layer_counter``;
* the handle's fp16 output is cast to the query's dtype, and its spike
  flags / tokens are stashed on the layer's ``FusedCacheWrapper`` for the
  promotion pipeline.

The model side follows the mlx-lm conventions the reference relies on:
``model(tokens, cache=caches)`` returns logits (B, L, vocab), each
attention layer calls ``keys, values = cache.update_and_fetch(k, v)`` and
then ``F.scaled_dot_product_attention`` (looked up on the module at call
time), RoPE reads ``cache.offset``, and ``len(model.layers)`` is the layer
count.  ``KVCache`` / ``make_prompt_cache`` are the standard fp16 cache used
for prefill.

One difference from the reference: when a ``PromotionPipeline`` is drained
through ``drain_spikes``, each layer's decode launch is ordered after that
layer's promotion copies (``PromotionPipeline.order``), because here the
copies are asynchronous device work rather than CPU stores into unified
memory.

Extension: ``generate_fused(..., graph=True)`` keeps the decode-step state
on the device (``_DeviceDecode``) and captures one whole model decode step
-- every layer's projections, RoPE, decode-buffer write, fused attention
(``fkv_attn_call_dev``: the decode count is read on the device), the device
spike drain of the previous step, and the greedy next token -- in a single
HIP graph that is replayed once per token.  The host then issues one launch
per token instead of the closure's per-layer Python and library calls.  The
model must accept a device tensor as ``cache.offset`` (its RoPE positions
computed as ``offset + arange(L)``).
"""

import shutil
import tempfile
import time
from typing import Optional

import numpy as np
import torch
import torch.nn.functional as F

from . import _lib
from .promotion import PromotionPipeline
from .tier_cache import MLXFoveatedKVCache, MLXTierConfig


# ---------------------------------------------------------------------------
# standard cache (prefill)
# ---------------------------------------------------------------------------

class KVCache:
    """Growing fp16/bf16 K, V cache with the mlx-lm interface the models
    use: ``update_and_fetch`` appends (B, H_kv, L, D) and returns all rows,
    ``state`` is (keys, values), ``offset`` the number of tokens held."""

    def __init__(self):
        self.keys = None
        self.values = None
        self.offset = 0

    def update_and_fetch(self, keys, values):
        if self.keys is None:
            self.keys, self.values = keys, values
        else:
            self.keys = torch.cat([self.keys, keys], dim=2)
            self.values = torch.cat([self.values, values], dim=2)
        self.offset += keys.shape[2]
        return self.keys, self.values

    @property
    def state(self):
        return self.keys, self.values


def make_prompt_cache(model) -> list:
    return [KVCache() for _ in range(len(model.layers))]


# ---------------------------------------------------------------------------
# fused SDPA closure
# ---------------------------------------------------------------------------

class _FusedSDPAState:
    """mlx_generate.py:42-54."""

    def __init__(self):
        self.original_sdpa = None
        self._installed = False
        self._fov_cache = None
        self._cpp_pipeline_handle = None
        self._layer_counter = 0
        self._n_layers = 0
        self._decode_step = 0
        self._fused_wrappers = None
        self._fused_disabled = False
        self._promotion = None  # pipeline whose flushed copies decode launches wait for
        self._dev = None  # _DeviceDecode while a device-count decode runs
        self._closure_s = 0.0  # host seconds spent in decode calls of the closure


_fused_state = _FusedSDPAState()


class FusedCacheWrapper:
    """mlx_generate.py:57-81: the cache object a model sees during fused
    decode.  ``update_and_fetch`` appends the new token to the layer's
    decode buffer and hands the same K, V back (the model needs tensors of
    the right shape; attention itself never reads them)."""

    def __init__(self, fov_layer, layer_idx: int):
        self.fov_layer = fov_layer
        self.layer_idx = layer_idx
        self.offset = fov_layer.total_tokens
        self._spike_flags = None
        self._spike_tokens = None
        self._far_idx_host = None
        self._dev = None  # _DeviceDecode: offset is then a device tensor

    @property
    def state(self):
        return self.fov_layer.near_k, self.fov_layer.near_v

    def update_and_fetch(self, keys, values):
        if self._dev is not None:  # row t of the fixed-capacity buffer, t on the device
            self.fov_layer.add_token_at(keys, values, self._dev.idx)
            return keys, values
        self.fov_layer.add_token(keys, values)
        self.offset += keys.shape[2]
        return keys, values

    def far_idx_device(self) -> torch.Tensor:
        """The layer's far_idx as a contiguous int32 device tensor (made once)."""
        if getattr(self, "_far_idx_dev", None) is None:
            self._far_idx_dev = self.fov_layer.far_idx.to(torch.int32).contiguous()
        return self._far_idx_dev

    def far_idx_host(self) -> np.ndarray:
        """int32 host copy of the layer's far_idx (B, H_kv, F), made once:
        the drain reads it every step and it never changes."""
        if self._far_idx_host is None:
            self._far_idx_host = np.ascontiguousarray(
                self.fov_layer.far_idx.detach().to("cpu", torch.int32).numpy())
        return self._far_idx_host


def _build_fused_interceptor(state: _FusedSDPAState):
    """mlx_generate.py:84-131.  ``scale`` is not forwarded to the kernel,
    which (like the reference's) always uses D^-1/2."""
    original = state.original_sdpa
    layers = state._fov_cache.layers
    n_layers = state._n_layers

    def interceptor(query, key, value, attn_mask=None, dropout_p=0.0, is_causal=False, scale=None, **kwargs):
        if query.dim() != 4 or query.shape[2] > 1:
            return original(query, key, value, attn_mask=attn_mask, dropout_p=dropout_p,
                            is_causal=is_causal, scale=scale, **kwargs)

        idx = state._layer_counter
        state._layer_counter = idx + 1
        if idx >= n_layers:
            idx = idx % n_layers

        layer = layers[idx]
        if layer is None or state._fused_disabled:
            return original(query, key, value, attn_mask=attn_mask, dropout_p=dropout_p,
                            is_causal=is_causal, scale=scale, **kwargs)

        t0 = time.perf_counter()
        dev = state._dev
        if dev is not None:
            out, flags, tokens = layer.attend_fused_dev(query, dev.n, dev.results(idx, query))
        else:
            promo = state._promotion
            if promo is not None:
                promo.order(idx)
            out, flags, tokens = layer.attend_fused_with_spikes(query)

        wrappers = state._fused_wrappers
        if wrappers is not None and idx < len(wrappers):
            w = wrappers[idx]
            if w is not None:
                w._spike_flags = flags
                w._spike_tokens = tokens

        if out.dtype != query.dtype:
            out = out.to(query.dtype)
        state._closure_s += time.perf_counter() - t0
        return out

    return interceptor


def install_fused_sdpa(fov_cache) -> None:
    """mlx_generate.py:134-161.  Loads the gfx950 library first, so a
    missing library raises here instead of on the first decode call."""
    if _fused_state._installed:
        raise RuntimeError("Fused SDPA already installed -- call uninstall_fused_sdpa() first")
    _lib.load()

    s = _fused_state
    s.original_sdpa = F.scaled_dot_product_attention
    s._fov_cache = fov_cache
    s._cpp_pipeline_handle = None
    s._layer_counter = 0
    s._n_layers = len(fov_cache.layers)
    s._decode_step = 0
    s._fused_wrappers = None
    s._fused_disabled = False
    s._promotion = None
    s._installed = True
    F.scaled_dot_product_attention = _build_fused_interceptor(s)


def uninstall_fused_sdpa() -> None:
    """mlx_generate.py:164-178: restore the original function and clear state."""
    s = _fused_state
    if not s._installed:
        return
    F.scaled_dot_product_attention = s.original_sdpa
    s.__init__()


def install_fused_attention(model, fov_cache) -> list:
    """mlx_generate.py:186-201: install the closure and return one
    ``FusedCacheWrapper`` per layer (None for empty layers), to be passed as
    the model's cache."""
    wrappers = [FusedCacheWrapper(layer, i) if layer is not None else None
                for i, layer in enumerate(fov_cache.layers)]
    install_fused_sdpa(fov_cache)
    _fused_state._fused_wrappers = wrappers
    return wrappers


def uninstall_fused_attention(model) -> None:
    """mlx_generate.py:204-206."""
    uninstall_fused_sdpa()


def _drain_into(pipeline, wrappers, step: int) -> None:
    """Hand every stashed (flags, tokens) pair to ``pipeline.drain_spikes``
    and clear the stash.  For this package's ``PromotionPipeline`` the
    spike arrays of all layers come to the host in one copy and the queued
    promotions are flushed once, after the last layer; with
    ``pipeline.device_drain`` set the drain and the row copies stay on the
    GPU (``drain_spikes_device``, no host round trip)."""
    ready = [w for w in (wrappers or [])
             if w is not None and w._spike_flags is not None and w._spike_tokens is not None]
    if pipeline is not None and ready:
        if isinstance(pipeline, PromotionPipeline) and getattr(pipeline, "device_drain", False):
            for w in ready:
                pipeline.drain_spikes_device(w.layer_idx, w._spike_flags.to(torch.int32).contiguous(),
                                             w._spike_tokens.to(torch.int32).contiguous(), w.far_idx_device(),
                                             step)
        elif isinstance(pipeline, PromotionPipeline):
            # every layer's flags and tokens (B,Hq[,K]) in one device-to-host copy
            parts = [t.to(torch.int32).reshape(-1) for w in ready for t in (w._spike_flags, w._spike_tokens)]
            host = torch.cat(parts).cpu().numpy()
            at = 0
            for w in ready:
                nf, nt = w._spike_flags.numel(), w._spike_tokens.numel()
                flags = host[at:at + nf].reshape(tuple(w._spike_flags.shape))
                tokens = host[at + nf:at + nf + nt]
                at += nf + nt
                pipeline.drain_spikes(w.layer_idx, flags, tokens, w.far_idx_host(), step, flush=False)
            pipeline.flush()
        else:
            for w in ready:
                pipeline.drain_spikes(w.layer_idx, w._spike_flags, w._spike_tokens,
                                      w.fov_layer.far_idx, step)
    for w in wrappers or []:
        if w is not None:
            w._spike_flags = None
            w._spike_tokens = None


def drain_spikes(wrappers: list, pipeline, decode_step: int) -> None:
    """mlx_generate.py:209-230: reset the layer counter, then drain the
    stashed spikes of the last step into ``pipeline`` (skipped when None)."""
    reset_fused_layer_counter()
    if pipeline is None:
        return
    if hasattr(pipeline, "order"):
        _fused_state._promotion = pipeline
    _drain_into(pipeline, wrappers, decode_step)


def reset_fused_layer_counter() -> None:
    """mlx_generate.py:233-259: start a new decode step; drains into the
    state's own pipeline handle when one is set."""
    s = _fused_state
    s._layer_counter = 0
    s._decode_step += 1
    if s._cpp_pipeline_handle is None:
        return
    _drain_into(s._cpp_pipeline_handle, s._fused_wrappers, s._decode_step)


# ---------------------------------------------------------------------------
# device-count decode (one HIP graph per model decode step)
# ---------------------------------------------------------------------------

class _DeviceDecode:
    """Decode-step state held in device memory, so that a model decode step
    reads no host value that changes from step to step and can be captured
    once in a HIP graph: the step t (int32; the device drain's step), the
    decode count t + 1 (int32; read by the attention kernel), the decode
    buffer row t (int64), each layer's RoPE offset prompt_len + t (int64,
    0-d, handed to the model as ``cache.offset``), and per-layer result
    tensors the kernel writes, so the next step's drain reads fixed
    addresses.  ``refresh`` derives everything from t at the start of a
    step; the step advances t at its end."""

    def __init__(self, wrappers, capacity: int, device):
        self.wrappers = wrappers
        self.t = torch.zeros(1, dtype=torch.int32, device=device)
        self.n = torch.ones(1, dtype=torch.int32, device=device)
        self.idx = torch.zeros(1, dtype=torch.int64, device=device)
        self._pos = {}
        self._base = {}
        self._out = {}
        self._spike_k = {}  # layer -> spike tokens per query head
        for w in wrappers:
            if w is None:
                continue
            base = int(w.offset)
            self._base[w.layer_idx] = base
            if base not in self._pos:
                self._pos[base] = torch.full((), base, dtype=torch.int64, device=device)
            w.fov_layer.reserve_decode(capacity)
            w.offset = self._pos[base]
            w._dev = self
            self._spike_k[w.layer_idx] = int(getattr(w.fov_layer, "spike_k", 1))

    def results(self, layer_idx: int, query):
        """The layer's (out, flags, tokens) tensors, made at its first call
        (outside any capture)."""
        r = self._out.get(layer_idx)
        if r is None:
            B, Hq, _, D = query.shape
            k = self._spike_k.get(layer_idx, 1)
            r = (torch.zeros((B, Hq, 1, D), dtype=torch.float16, device=query.device),
                 torch.zeros((B, Hq), dtype=torch.int32, device=query.device),
                 torch.zeros((B, Hq) if k == 1 else (B, Hq, k), dtype=torch.int32, device=query.device))
            self._out[layer_idx] = r
        return r

    def refresh(self) -> None:
        torch.add(self.t, 1, out=self.n)
        self.idx.copy_(self.t)
        for base, p in self._pos.items():
            torch.add(self.idx[0], base, out=p)

    def drain(self, pipeline) -> None:
        """The device drain of the previous step's spikes, every layer with
        results, at step t (as ``_drain_into`` with ``device_drain``)."""
        for w in self.wrappers:
            if w is None or w.layer_idx not in self._out:
                continue
            _, flags, tokens = self._out[w.layer_idx]
            pipeline.drain_spikes_device(w.layer_idx, flags, tokens, w.far_idx_device(), self.t)

    def close(self, steps: int) -> None:
        """Back to host-count decode after ``steps`` model calls: offsets and
        decode-buffer counts become host ints again."""
        for w in self.wrappers:
            if w is None:
                continue
            w._dev = None
            w.offset = self._base[w.layer_idx] + steps
            w.fov_layer._decode.n = steps
            w.fov_layer._next_pos += steps


# ---------------------------------------------------------------------------
# generation
# ---------------------------------------------------------------------------

def _model_device(model):
    for p in model.parameters():
        return p.device
    return torch.device("cuda")


def prefill_and_compress(model, tokens: torch.Tensor, cfg: Optional[MLXTierConfig] = None):
    """mlx_generate.py:390-416 -> (fov_cache, prefill_logits, std_caches)."""
    cfg = cfg or MLXTierConfig()
    std_caches = make_prompt_cache(model)
    with torch.no_grad():
        prefill_logits = model(tokens, cache=std_caches)
    fov_cache = MLXFoveatedKVCache(cfg)
    for i, c in enumerate(std_caches):
        k, v = c.state
        if k is not None:
            fov_cache.update(k, v, i)
    fov_cache.compress()
    return fov_cache, prefill_logits, std_caches


def _next_token(logits, temp):
    if temp == 0:
        return torch.argmax(logits, dim=-1)
    return torch.multinomial(torch.softmax(logits.float() / temp, dim=-1), 1).reshape(-1)


def generate_fused(model, tokenizer, prompt: str, max_tokens: int = 100,
                   cfg: Optional[MLXTierConfig] = None, disk_archive_dir: Optional[str] = None,
                   temp: float = 0.0, enable_promotion: bool = True, device_drain: bool = False,
                   graph: bool = False):
    """mlx_generate.py:266-387: prefill, compress, move archives to disk,
    register them and the handles with a ``PromotionPipeline``, then decode
    with the closure installed.  Returns (text, stats).  ``device_drain``
    (extension): drain and promote on the GPU after each step instead of
    reading the spike outputs back (same promotions).  ``graph``
    (extension, greedy only, implies ``device_drain``): capture one whole
    model decode step in a HIP graph and replay it per token (same tokens
    and promotions as the eager loop).  ``stats["host_us_per_layer"]`` is
    the host time spent issuing the decode steps (drain + model call, or the
    graph replay) per model call and layer."""
    from .disk_archive import offload_cache_to_disk

    if graph and temp != 0:
        raise ValueError("graph decode is greedy: it needs temp=0")
    dev = _model_device(model)
    tokens = torch.tensor(tokenizer.encode(prompt), dtype=torch.long, device=dev).reshape(1, -1)

    t0 = time.perf_counter()
    fov_cache, prefill_logits, _ = prefill_and_compress(model, tokens, cfg)
    t_prefill = time.perf_counter() - t0
    mem_before = fov_cache.memory_bytes()

    own_dir = disk_archive_dir is None
    if own_dir:
        disk_archive_dir = tempfile.mkdtemp(prefix="foveated_fused_")
    disk_archives = offload_cache_to_disk(fov_cache, disk_archive_dir)
    mem_after = fov_cache.memory_bytes()

    pipeline = None
    if enable_promotion:
        pipeline = PromotionPipeline(len(fov_cache.layers), spike_k=int(getattr(cfg, "spike_k", 1)) if cfg else 1)
        pipeline.device_drain = bool(device_drain or graph)
        for i, layer in enumerate(fov_cache.layers):
            if layer is None:
                continue
            layer._ensure_kcache()
            handle = layer._kcache.get("cpp_handle")
            if handle is not None and hasattr(handle, "get_blob_info"):
                pipeline.register_blob(i, handle.get_blob_info())
            if i < len(disk_archives) and disk_archives[i] is not None:
                a = disk_archives[i]
                pipeline.register_archive(i, a.path_k, a.path_v, a.H_kv, a.S_arc, a.D, a.idx)

    wrappers = install_fused_attention(model, fov_cache)
    eos = getattr(tokenizer, "eos_token_id", None)
    generated = []
    next_logits = prefill_logits[:, -1, :]
    torch.cuda.synchronize(dev)
    t_dec = time.perf_counter()
    t_issue = 0.0
    calls = 0
    _fused_state._closure_s = 0.0
    try:
        with torch.no_grad():
            if graph:
                generated, calls, t_issue = _decode_graph(model, wrappers, pipeline, next_logits, max_tokens,
                                                          eos, dev)
            else:
                for step in range(max_tokens):
                    tok = _next_token(next_logits, temp)
                    token_id = int(tok.item())
                    if token_id == eos:
                        break
                    generated.append(token_id)
                    t0 = time.perf_counter()
                    drain_spikes(wrappers, pipeline, step)
                    next_logits = model(tok.reshape(1, 1), cache=wrappers)[:, -1, :]
                    t_issue += time.perf_counter() - t0
                    calls += 1
        torch.cuda.synchronize(dev)
    finally:
        t_decode = time.perf_counter() - t_dec
        closure_s = _fused_state._closure_s
        uninstall_fused_attention(model)
        if pipeline is not None:
            pipeline.stop()
        shutil.rmtree(disk_archive_dir, ignore_errors=True)
    n_fused = sum(1 for w in wrappers if w is not None)

    mb = 1024 * 1024
    stats = {
        "prompt_tokens": tokens.shape[1],
        "generated_tokens": len(generated),
        "fused_kernel": True,
        "disk_offloaded": True,
        "prefill_time_s": t_prefill,
        "decode_time_s": t_decode,
        "tokens_per_second": len(generated) / max(t_decode, 1e-6),
        "graph": bool(graph),
        "model_calls": calls,
        "host_us_per_layer": t_issue / max(calls * n_fused, 1) * 1e6,
        # the closure's own share (layer lookup, library call, result
        # tensors, spike stash); a replayed graph runs no closure
        "closure_us_per_layer": None if graph else closure_s / max(calls * n_fused, 1) * 1e6,
        "mem_quantized_mb": mem_before["total_quantized"] / mb,
        "mem_archive_before_mb": mem_before["archive"] / mb,
        "mem_archive_after_mb": mem_after["archive"] / mb,
        "mem_saved_mb": (mem_before["archive"] - mem_after["archive"]) / mb,
    }
    if pipeline is not None:
        stats.update(pipeline.get_stats())
    return tokenizer.decode(generated), stats


def _decode_graph(model, wrappers, pipeline, next_logits, max_tokens, eos, dev, chunk=16):
    """Greedy decode of up to ``max_tokens`` tokens with the step state on the
    device.  Steps 0 and 1 run eagerly (they size every workspace and make
    the drain's device tables, which must not happen under capture); step 2
    is captured in one HIP graph and replayed for every later step.  Token
    t + 1 = argmax of model call t is written into a device history; with an
    EOS id the history is read every ``chunk`` steps and the tokens from the
    first EOS on are dropped (the eager loop stops there), so the result is
    the eager loop's.  -> (tokens, model calls, host issue seconds)."""
    s = _fused_state
    dd = _DeviceDecode(wrappers, max(max_tokens, 1), dev)
    s._dev = dd
    hist = torch.zeros(max_tokens + 1, dtype=torch.int64, device=dev)
    hist[0:1].copy_(torch.argmax(next_logits, dim=-1))

    def step():
        s._layer_counter = 0
        dd.refresh()
        if pipeline is not None:
            dd.drain(pipeline)
        tok = hist.index_select(0, dd.idx).view(1, 1)
        logits = model(tok, cache=wrappers)[:, -1, :]
        hist.index_copy_(0, dd.idx + 1, torch.argmax(logits, dim=-1))
        dd.t.add_(1)

    calls, t_issue, n_tok = 0, 0.0, max_tokens
    g = None
    main = torch.cuda.current_stream(dev)
    side = torch.cuda.Stream(device=dev)  # the eager steps run here, as before any capture
    try:
        while calls < n_tok:
            if eos is not None and calls % chunk == 0:
                known = hist[: calls + 1].tolist()
                if eos in known:
                    n_tok = known.index(eos)
                    break
            if calls >= 2 and g is None:
                main.wait_stream(side)
                torch.cuda.synchronize(dev)
                g = torch.cuda.CUDAGraph()
                with torch.cuda.graph(g):
                    step()
            t0 = time.perf_counter()
            if g is None:
                side.wait_stream(main)
                with torch.cuda.stream(side):
                    step()
                main.wait_stream(side)
            else:
                g.replay()
            t_issue += time.perf_counter() - t0
            calls += 1
        known = hist[: min(calls, n_tok) + 1].tolist()
    finally:
        torch.cuda.synchronize(dev)
        s._dev = None
        dd.close(calls)
    if eos is not None and eos in known:
        n_tok = min(n_tok, known.index(eos))
    return known[: min(n_tok, calls)], calls, t_issue
